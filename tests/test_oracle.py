"""Pins the CPU oracle (oracle/vmlm_oracle.c) before it is trusted as the
checker of the HIP path.

Each test names what it pins and against what: the reference's own
known-answer tests and fixtures (copied under tests/golden/reference/),
closed forms, invariants, or brute-force float64. Every check is chosen so a
plausible restatement mistake (dropped term, wrong sign/index/constant,
transposed operand) fails it.
"""
import math
import struct

import numpy as np
import pytest

REF = "reference"


def f64_rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b) / np.maximum(np.abs(b), 1e-300)


# ---------------------------------------------------------------- exp_f
def test_exp_f_reference_kats(oracle):
    """tests/src/main.rs:166-199: exp_f(0)==1 exactly; exp_f(-88) is the
    subnormal 6.054602e-39 (within 1e-6 rel); no NaN on the edge list;
    monotone on [-20,20]."""
    assert oracle.exp_f(0.0) == 1.0
    v = oracle.exp_f(-88.0)
    assert v > 0 and abs(v - math.exp(-88.0)) / math.exp(-88.0) < 1e-6
    for x in [-1e30, -88.0, -87.9, -87.34, -87.0, -1.0, -0.0, 0.0, 1e-30, 1.0, 88.0, 1e30]:
        assert not math.isnan(oracle.exp_f(x))
    xs = (-20.0 + 40.0 * np.arange(200000, dtype=np.float32) / np.float32(199999.0)).astype(
        np.float32)
    ys = oracle.vmap("exp", xs)
    assert np.all(np.diff(ys.astype(np.float64)) >= 0)


def test_nan_propagates_like_rust(oracle):
    """sys/src/math/mod.rs:133 converts with Rust's `n as i32`, which maps NaN
    to 0: exp_f(NaN) = p * 2^0 with p NaN, so NaN (not the underflow branch's
    0.0); tanh / sigmoid / SiLU of NaN are NaN; sin/cos of NaN are NaN."""
    nan = float("nan")
    assert math.isnan(oracle.exp_f(nan))
    x = np.array([nan, -nan], np.float32)
    for name in ("exp", "tanh", "sin", "cos"):
        assert np.all(np.isnan(oracle.vmap(name, x))), name
    for kind in (2, 3, 4):  # SiLU, sigmoid, tanh
        assert np.all(np.isnan(oracle.act(x, kind))), kind


def test_exp_f_full_domain_sweep(oracle):
    """tests/src/main.rs:84-160: max rel <= 1e-6 over the normal-result range
    of [-88, 88] (reference measured 7.91e-8); subnormal results within the
    representation limit. Dropping LN2_LO or perturbing a coefficient fails."""
    x = np.linspace(-88.0, 88.0, 1_000_001).astype(np.float32)
    # densify around multiples of ln2 (the reduction seams)
    seams = (np.arange(-127, 128) * np.log(2.0))
    x = np.concatenate([x, (seams[:, None] + np.linspace(-1e-4, 1e-4, 41)[None, :]).ravel()
                        .astype(np.float32)])
    x = x[(x >= -88.0) & (x <= 88.0)]
    y = oracle.vmap("exp", x).astype(np.float64)
    r = np.exp(x.astype(np.float64))
    normal = r >= 2.0 ** -126
    assert f64_rel(y[normal], r[normal]).max() <= 1e-6
    sub = ~normal
    assert np.all(np.abs(y[sub] - r[sub]) <= 2.0 ** -149 + 1e-6 * r[sub])


def test_round_floor(oracle):
    """sys/src/math/mod.rs:68-71 round-half-even for |v| < 2^22;
    ops/src/kernels.rs:216-223 floor (negatives go down)."""
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.uniform(-4e6, 4e6, 20000), np.arange(-10, 10) + 0.5]).astype(
        np.float32)
    assert np.array_equal(oracle.vmap("round", v), np.rint(v))
    f = np.concatenate([rng.uniform(-1e6, 1e6, 20000), [-0.5, -1.0, 0.0, 2.999, -2.0001]]
                       ).astype(np.float32)
    assert np.array_equal(oracle.vmap("floor", f), np.floor(f))


def test_sin_cos_accuracy(oracle):
    """ops/src/kernels.rs:189: 3.1e-8 on [-pi/4, pi/4] (+ f32 output
    rounding); over [-100, 100] the n*PI2_HI product rounds, which the
    reference documents as ~ulp(x) (:96-101), so the sweep bound is 5e-6.
    At x = n*pi/2 + 0.3 with n a power of two the product is exact and the
    error must be ~1e-7: a sign error in PI2_MID costs 2*n*4.4e-8 there
    (3.6e-4 at n=4096)."""
    x = np.linspace(-math.pi / 4, math.pi / 4, 200001).astype(np.float32)
    x64 = x.astype(np.float64)
    assert np.abs(oracle.vmap("sin", x) - np.sin(x64)).max() <= 1e-7
    assert np.abs(oracle.vmap("cos", x) - np.cos(x64)).max() <= 1e-7
    x = np.linspace(-100, 100, 400001).astype(np.float32)
    x64 = x.astype(np.float64)
    assert np.abs(oracle.vmap("sin", x) - np.sin(x64)).max() <= 5e-6
    assert np.abs(oracle.vmap("cos", x) - np.cos(x64)).max() <= 5e-6
    n = 2.0 ** np.arange(0, 13)
    x = (n * (np.pi / 2) + 0.3).astype(np.float32)
    x64 = x.astype(np.float64)
    assert np.abs(oracle.vmap("sin", x) - np.sin(x64)).max() <= 2e-7
    assert np.abs(oracle.vmap("cos", x) - np.cos(x64)).max() <= 2e-7
    assert oracle.sin_f(0.0) == 0.0 and oracle.cos_f(0.0) == 1.0


def test_ln_tanh(oracle):
    """ops/src/kernels.rs:240-255 ln_f and :58-67 tanh_f vs float64."""
    x = np.exp(np.linspace(-60, 60, 100001)).astype(np.float32)
    y = oracle.vmap("ln", x)
    assert np.abs(y - np.log(x.astype(np.float64))).max() <= 2e-5  # |ln x| <= 60
    assert f64_rel(y[np.abs(np.log(x)) > 1], np.log(x[np.abs(np.log(x)) > 1].astype(
        np.float64))).max() <= 3e-7
    assert oracle.ln_f(0.0) == -88.0 and oracle.ln_f(-1.0) == -88.0
    t = np.linspace(-20, 20, 200001).astype(np.float32)
    th = oracle.vmap("tanh", t)
    assert np.abs(th - np.tanh(t.astype(np.float64))).max() <= 2e-7
    assert oracle.tanh_f(15.5) == 1.0 and oracle.tanh_f(-15.5) == -1.0


def test_activations(oracle):
    """ops/src/kernels.rs:27-52 act_scalar kinds vs their definitions."""
    x = np.linspace(-12, 12, 4001).astype(np.float32)
    x64 = x.astype(np.float64)
    silu = oracle.vmap(102, x)
    assert np.abs(silu - x64 / (1 + np.exp(-x64))).max() <= 3e-6
    sig = oracle.vmap(103, x)
    assert np.abs(sig - 1 / (1 + np.exp(-x64))).max() <= 2e-7
    relu = oracle.vmap(100, x)
    assert np.array_equal(relu, np.maximum(x, 0))
    r2 = oracle.vmap(105, x)
    assert np.array_equal(r2, (np.maximum(x, 0) * np.maximum(x, 0)).astype(np.float32))
    gelu = oracle.vmap(101, x)
    ref = 0.5 * x64 * (1 + np.tanh(0.7978846 * (x64 + 0.044715 * x64 ** 3)))
    assert np.abs(gelu - ref).max() <= 5e-6


def test_bf16_roundtrip(oracle):
    """tensor/src/dtype.rs:40-51: RNE to bf16; widen is a 16-bit shift."""
    rng = np.random.default_rng(1)
    v = rng.standard_normal(20000).astype(np.float32)
    h = oracle.f32_to_bf16(v)
    for i in range(0, 20000, 997):
        assert h[i] == oracle.lib().vo_f32_to_bf16(float(v[i]))
    w = oracle.bf16_to_f32(h)
    assert np.all(np.abs(w - v) <= np.abs(v) * 2.0 ** -8)
    # exactness: values with <= 8 significant bits are unchanged
    ints = np.arange(-256, 257, dtype=np.float32)
    assert np.array_equal(oracle.bf16_to_f32(oracle.f32_to_bf16(ints)), ints)
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1+2^-7 -> 1
    assert oracle.bf16_to_f32(oracle.f32_to_bf16(np.float32([1 + 2 ** -8])))[0] == 1.0


# ---------------------------------------------------------------- GEMMs
GEMM_SHAPES = [(4, 8, 8), (1, 1, 64), (1, 32, 64), (1, 10, 32), (8, 8, 512),
               (512, 512, 512), (3, 5, 7), (5, 3, 9), (17, 23, 31), (64, 64, 64),
               (16, 1, 16), (1, 16, 16), (16, 16, 1)]


def _ref_inputs(m, n, k):
    i = np.arange(m * k)
    a = ((i * 37 % 100).astype(np.float32) / np.float32(50.0) - np.float32(1.0)).astype(
        np.float32).reshape(m, k)
    i = np.arange(n * k)
    b = ((i * 53 % 100).astype(np.float32) / np.float32(50.0) - np.float32(1.0)).astype(
        np.float32).reshape(n, k)
    return a, b


def _naive_f32(a, b):
    """tests/src/main.rs:283-296 naive: f32 products summed left to right."""
    m, n = a.shape[0], b.shape[0]
    c = np.empty((m, n), np.float32)
    for i in range(m):
        prods = (a[i][None, :] * b).astype(np.float32)  # [n, k] f32 products
        c[i] = np.add.accumulate(prods, axis=1, dtype=np.float32)[:, -1]
    return c


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_nt_reference_shapes(oracle, m, n, k):
    """tests/src/main.rs:338-344: the 13 regression shapes with the
    reference's inputs, maxerr < 1e-3 vs naive; where the reference dispatch
    takes the scalar path (m<8 or n<8) the result must equal naive bitwise."""
    a, b = _ref_inputs(m, n, k)
    c = oracle.gemm_nt(a, b)
    naive = _naive_f32(a, b)
    assert np.abs(c - naive).max() < 1e-3
    assert np.abs(c - a.astype(np.float64) @ b.astype(np.float64).T).max() < 1e-3
    if m < 8 or n < 8:
        assert np.array_equal(c.view(np.uint32), naive.view(np.uint32))


def test_gemm_nt_acc_and_nn(oracle):
    rng = np.random.default_rng(2)
    a = rng.standard_normal((9, 33)).astype(np.float32)
    b = rng.standard_normal((12, 33)).astype(np.float32)
    c0 = rng.standard_normal((9, 12)).astype(np.float32)
    c = oracle.gemm_nt(a, b, c0, acc=True)
    ref = c0.astype(np.float64) + a.astype(np.float64) @ b.astype(np.float64).T
    assert np.abs(c - ref).max() < 1e-4
    # NN (ops/src/kernels.rs:383-419) is the scalar chain: bitwise naive on B^T
    bn = rng.standard_normal((33, 12)).astype(np.float32)
    cn = oracle.gemm(a, bn)
    assert np.array_equal(cn, _naive_f32(a, np.ascontiguousarray(bn.T)))


def test_gemm_nt_int8_kat(oracle, golden_dir):
    """tools/p13_q8_check.py:42-47 with its committed inputs
    (examples/p13/q8_*): A=[1,2,3,4], W=[[1,0,-1,0],[0,2,0,-2]],
    scale=[0.5,0.25] -> [[-1,-1]] exactly."""
    d = golden_dir / REF
    a = np.fromfile(d / "q8_a.f32", np.float32).reshape(1, 4)
    w = np.fromfile(d / "q8_w.i8", np.int8).reshape(2, 4)
    s = np.fromfile(d / "q8_scale.f32", np.float32)
    assert np.array_equal(a, [[1, 2, 3, 4]])
    assert np.array_equal(w, [[1, 0, -1, 0], [0, 2, 0, -2]])
    c = oracle.gemm_nt_int8(a, w, s)
    assert np.array_equal(c, np.float32([[-1.0, -1.0]]))


def test_gemm_nt_int8_exact_and_random(oracle):
    """sparrow/examples/int8_one.sparrow: w = q/64 exactly representable,
    scale = 1/64 -> int8 path equals the f32 result exactly for small-integer
    activations; random shapes with K tails vs float64. A transposed weight or
    a missing / per-column scale fails the float64 check."""
    rng = np.random.default_rng(3)
    for (m, n, k) in [(1, 7, 13), (3, 16, 64), (16, 40, 2305), (2, 5, 1)]:
        q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
        s = np.full(n, 1 / 64, np.float32)
        c = oracle.gemm_nt_int8(a, q, s)
        exact = (a.astype(np.float64) @ q.astype(np.float64).T) / 64.0
        assert np.array_equal(c.astype(np.float64), exact)
        a = rng.standard_normal((m, k)).astype(np.float32)
        s = (np.abs(rng.standard_normal(n)) * 0.02 / 127 + 1e-6).astype(np.float32)
        c = oracle.gemm_nt_int8(a, q, s)
        ref = (a.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
        rms = np.sqrt(np.mean(ref ** 2))
        assert np.abs(c - ref).max() <= 1e-5 * rms


def test_gemm_nt_bf16(oracle):
    """ops/src/kernels.rs:1199-1227 vs float64; K=1 is the single f32
    product (the scalar tail: 0 + a*b)."""
    rng = np.random.default_rng(4)
    for (m, n, k) in [(1, 9, 1), (2, 17, 16), (5, 33, 37), (16, 64, 512)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = oracle.f32_to_bf16(rng.standard_normal((n, k)).astype(np.float32))
        c = oracle.gemm_nt_bf16(a, b)
        ref = a.astype(np.float64) @ oracle.bf16_to_f32(b).astype(np.float64).T
        if k == 1:
            assert np.array_equal(c, (a * oracle.bf16_to_f32(b).T).astype(np.float32))
        assert np.abs(c - ref).max() <= 2e-6 * max(1.0, np.sqrt(k))


# ---------------------------------------------------------------- row ops
def test_rmsnorm(oracle):
    """ops/src/kernels.rs:1346-1368: constant row c -> c/sqrt(c^2+eps)*g;
    random rows vs float64."""
    g = np.linspace(0.5, 1.5, 64).astype(np.float32)
    x = np.full((2, 64), 3.0, np.float32)
    x[1] = -2.0
    y = oracle.rmsnorm(x, g, 1e-5)
    for r, c in [(0, 3.0), (1, -2.0)]:
        assert np.allclose(y[r], c / np.sqrt(c * c + 1e-5) * g, rtol=1e-6, atol=0)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 2304)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 2304).astype(np.float32)
    y = oracle.rmsnorm(x, g, 1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5) * g
    assert np.abs(y - ref).max() <= 2e-6 * np.abs(ref).max()


def test_softmax(oracle):
    """ops/src/kernels.rs:1388-1414: rows sum to 1; causal tail exactly 0;
    vs float64; the p13_kv_probe scores {17,39,61} give exactly 1.0 on the
    max term in f32 (tools/p13_kv_probe.py:98-103)."""
    rng = np.random.default_rng(6)
    p = rng.standard_normal((6, 10)).astype(np.float32) * 3
    s = oracle.softmax(p, causal=True)
    for r in range(6):
        assert np.all(s[r, r + 1:] == 0.0)
        assert abs(s[r, :r + 1].sum(dtype=np.float64) - 1) < 1e-6
        e = np.exp(p[r, :r + 1].astype(np.float64) - p[r, :r + 1].max())
        assert np.abs(s[r, :r + 1] - e / e.sum()).max() < 1e-6
    one = oracle.softmax(np.float32([[17, 39, 61]]))
    assert one[0, 2] == 1.0


def test_kv_probe_kat(oracle, golden_dir):
    """tools/p13_kv_probe.py:40-49,92-105 on its committed inputs
    (examples/p13/{kk,vv,qq}.f32): scores (5, 11, 17) from an NN GEMM against
    the transposed cache, softmax, then the NT context GEMM."""
    d = golden_dir / REF
    K = np.fromfile(d / "kk.f32", np.float32).reshape(3, 2)
    V = np.fromfile(d / "vv.f32", np.float32).reshape(3, 2)
    Q = np.fromfile(d / "qq.f32", np.float32).reshape(1, 2)
    sc = oracle.gemm(Q, np.ascontiguousarray(K.T))
    assert np.array_equal(sc, np.float32([[5, 11, 17]]))
    sm = oracle.softmax(sc)
    ctx = oracle.gemm_nt(sm, np.ascontiguousarray(V.T))
    e = np.exp(np.array([5, 11, 17], np.float64) - 17)
    ref = (e / e.sum()) @ V.astype(np.float64)
    assert np.abs(ctx[0] - ref).max() < 1e-4


def test_rope(oracle):
    """core/src/interp.rs:1159-1223: position 0 is the identity bitwise;
    pair norms are preserved; angles match pos*theta^(-2i/hd) in float64;
    odd hd and theta<=0 are guard failures (exit 9)."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 64)).astype(np.float32)
    assert np.array_equal(oracle.rope(x, 10000.0, 0), x)
    x = rng.standard_normal((40, 64)).astype(np.float32)
    pos0 = 1000
    y = oracle.rope(x, 10000.0, pos0)
    half = 32
    i = np.arange(half, dtype=np.float64)
    inv = 10000.0 ** (-2 * i / 64)
    pos = pos0 + np.arange(40, dtype=np.float64)[:, None]
    ang = pos * inv[None, :]
    x1, x2 = x[:, :half].astype(np.float64), x[:, half:].astype(np.float64)
    r1 = x1 * np.cos(ang) - x2 * np.sin(ang)
    r2 = x1 * np.sin(ang) + x2 * np.cos(ang)
    ref = np.concatenate([r1, r2], 1)
    assert np.abs(y - ref).max() < 2e-4  # f32 angle reduction at pos ~1e3
    n0 = np.hypot(x1, x2)
    n1 = np.hypot(y[:, :half].astype(np.float64), y[:, half:].astype(np.float64))
    assert np.abs(n1 - n0).max() < 1e-5
    with pytest.raises(ValueError):
        oracle.rope(np.zeros((1, 63), np.float32), 10000.0, 0)
    with pytest.raises(ValueError):
        oracle.rope(np.zeros((1, 64), np.float32), 0.0, 0)


def test_emb_guards_and_widen(oracle, golden_dir):
    """core/src/interp.rs:1351-1436: exact bf16 widen; negative, NaN,
    out-of-range and fractional row indices are guard failures (exit 9).
    The f32 table fixture of tools/p13_emb_check.py is read back exactly."""
    rng = np.random.default_rng(8)
    tab = oracle.f32_to_bf16(rng.standard_normal((5, 16)).astype(np.float32))
    st, row = oracle.emb_bf16(tab, 3.0)
    assert st == 0 and np.array_equal(row, oracle.bf16_to_f32(tab[3]))
    for bad in [-1.0, float("nan"), 5.0, 2.5, 1e9]:
        st, _ = oracle.emb_bf16(tab, bad)
        assert st == 9
    t32 = np.fromfile(golden_dir / REF / "table_f32.f32", np.float32).reshape(3, 4)
    out = np.empty(4, np.float32)
    assert oracle.lib().vo_emb_f32(out, t32, 3, 4, 2.0) == 0
    assert np.array_equal(out, t32[2])


def test_topk_idx(oracle):
    """core/src/interp.rs:1649-1681: strict `>` -> lowest index wins ties."""
    assert oracle.topk_idx(np.float32([3, 1, 5, 2, 4, 0.5, 6, 1.5]))[1] == 6.0
    assert oracle.topk_idx(np.float32([2, 7, 7, 1]))[1] == 1.0
    assert oracle.topk_idx(np.zeros(9, np.float32))[1] == 0.0
    assert oracle.topk_idx(np.float32([-5, -1, -1]))[1] == 1.0


# ---------------------------------------------------------------- B1
def test_prng_kats(oracle):
    """examples/p17_infer/ref_L2_d16.txt:9 (the reference engine's printed
    values): neuron_seed(0,0), neuron_conn_src(0,0,0,16,8), neuron_rand(12345,7)."""
    assert oracle.neuron_seed(0, 0) == 4245456706
    assert oracle.neuron_conn_src(0, 0, 0, 16, 8) == 8
    assert oracle.neuron_rand(12345, 7) == 2955612665


def _read_p17_dump(path):
    """tools/p17_infer_ref.py:200-243 dump layout."""
    b = path.read_bytes()
    o = 0

    def u32():
        nonlocal o
        v = struct.unpack_from("<I", b, o)[0]
        o += 4
        return v

    def f32s(n):
        nonlocal o
        v = np.frombuffer(b, np.float32, n, o).copy()
        o += 4 * n
        return v

    nl, d, k0, k, seq, vocab, ntok = (u32() for _ in range(7))
    toks = [u32() for _ in range(ntok)]
    emb = f32s(vocab * d)
    h0 = f32s(seq * d)
    layers = []
    for _ in range(nl):
        _wq, _wk = f32s(d * d), f32s(d * d)
        wv, wo, w, src = f32s(d * d), f32s(d * d), f32s(d * k0), f32s(d * k0)
        layers.append((wv, wo, w, src))
    layer_in = [f32s(seq * d) for _ in range(nl)]
    final = f32s(seq * d)
    assert o == len(b)
    return dict(nl=nl, d=d, k0=k0, k=k, seq=seq, toks=toks, emb=emb, h0=h0, layers=layers,
                layer_in=layer_in, final=final)


@pytest.mark.parametrize("name", ["dump_L2_d16_k08_k3_s3.bin", "dump_L3_d64_k020_k8_s5.bin"])
def test_p17_dump_replay_bitwise(oracle, golden_dir, name):
    """examples/p17_infer dumps written by the reference engine: (1) every
    dumped src equals neuron_conn_src (C1 of tools/p17_infer_ref.py); (2) the
    forward replayed from oracle pieces -- scalar-path GEMM_NT (m=1), the
    first-term-assigned gather contract over the top-k connections, f32
    residual adds -- reproduces every per-layer input and the final output
    BITWISE (C2/C3)."""
    D = _read_p17_dump(golden_dir / REF / name)
    d, k0, k, seq = D["d"], D["k0"], D["k"], D["seq"]
    h = D["h0"].reshape(seq, d).copy()
    for li, (wv, wo, w, src) in enumerate(D["layers"]):
        srcu = src.astype(np.uint32)
        want = np.array([[oracle.neuron_conn_src(li, i, j, d, k0) for j in range(k0)]
                         for i in range(d)], np.uint32).ravel()
        assert np.array_equal(srcu, want)
        assert np.array_equal(h.ravel().view(np.uint32), D["layer_in"][li].view(np.uint32))
        W = w.reshape(d, k0)
        S = srcu.reshape(d, k0)
        newh = np.empty_like(h)
        for t in range(seq):
            v = oracle.gemm_nt(h[t][None, :], wv.reshape(d, d))
            a = oracle.gemm_nt(v, wo.reshape(d, d))
            u = oracle.ew_op(h[t][None, :], a, 20)[0]
            # top-k by |w*u[src]|, ties keep the lower j, applied in ascending j
            strength = np.abs((W * u[S]).astype(np.float32))
            sel = np.zeros((d, k), np.int64)
            for i in range(d):
                order = sorted(range(k0), key=lambda j: (-float(strength[i, j]), j))
                sel[i] = sorted(order[:k])
            wk = np.take_along_axis(W, sel, 1).astype(np.float32)
            sk = np.take_along_axis(S, sel, 1).astype(np.uint32)
            y = oracle.b1_forward_t8(wk, sk, u[:, None].copy(), 1)[:, 0]
            newh[t] = oracle.ew_op(u, y, 20)
        h = newh
    assert np.array_equal(h.ravel().view(np.uint32), D["final"].view(np.uint32))


def test_b1_t8_contract(oracle):
    """ops/src/kernels.rs:1850-1862: first term assigned (so all -0.0 terms
    give -0.0, which an accumulator started at +0.0 would lose), j
    ascending; vs float64 on random data; zero padding columns untouched."""
    w = np.float32([[-1.0, -2.0]])
    src = np.uint32([[0, 1]])
    xt = np.float32([[0.0, 0.0], [0.0, 0.0]])  # [d=2][t8=2]
    yt = oracle.b1_forward_t8(w, src, xt, 2)
    assert np.all(np.signbit(yt))
    rng = np.random.default_rng(9)
    n, k0, T, t8 = 64, 32, 13, 16
    w = (rng.standard_normal((n, k0)) / np.sqrt(k0)).astype(np.float32)
    src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
    x = rng.standard_normal((T, n)).astype(np.float32)
    xt = oracle.transpose_t8(x, t8)
    assert np.all(xt[:, T:] == 0)
    yt = oracle.b1_forward_t8(w, src, xt, T)
    ref = np.einsum("ij,tij->it", w.astype(np.float64), x.astype(np.float64)[:, src])
    assert np.abs(yt[:, :T] - ref).max() < 1e-5
    y = oracle.transpose_t8_back(yt, T)
    assert np.array_equal(y, yt[:, :T].T)


def test_b1_forward_fold(oracle):
    """ops/src/kernels.rs:1773-1804 (8-lane fold) vs float64 for k0=32 and a
    tail k0=37; ops/src/kernels.rs:2720-2800 packed rows for k0 in {1,4,8}.
    The reference's k0==2 packed branch sums the two rows sharing a 128-bit
    half; the restatement reproduces that (rows i and i+1 both get the pair
    sum), recorded as a reference defect."""
    rng = np.random.default_rng(10)
    n = 24
    x = rng.standard_normal(n).astype(np.float32)
    for k0 in [1, 4, 8, 32, 37]:
        w = rng.standard_normal((n, k0)).astype(np.float32)
        src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
        y = oracle.b1_forward(w, src, x)
        ref = (w.astype(np.float64) * x.astype(np.float64)[src]).sum(1)
        assert np.abs(y - ref).max() < 1e-5
    w = rng.standard_normal((n, 2)).astype(np.float32)
    src = rng.integers(0, n, size=(n, 2)).astype(np.uint32)
    y = oracle.b1_forward(w, src, x)
    rows = (w * x[src]).astype(np.float32)
    pair = rows[0::2].sum(1) + rows[1::2].sum(1)
    assert np.allclose(y[0::2], pair, atol=1e-6) and np.allclose(y[1::2], pair, atol=1e-6)


# ---------------------------------------------------------------- attention
def _attn_f64(q, k, v, H, theta, causal):
    S, W = q.shape
    hd = W // H
    half = hd // 2
    i = np.arange(half, dtype=np.float64)
    ang = np.arange(S, dtype=np.float64)[:, None] * (theta ** (-2 * i / hd))[None, :]
    c, s = np.cos(ang), np.sin(ang)

    def rot(x):
        x1, x2 = x[:, :half], x[:, half:]
        return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], 1)

    out = np.empty((S, W))
    for h in range(H):
        sl = slice(h * hd, (h + 1) * hd)
        qh, kh, vh = rot(q[:, sl].astype(np.float64)), rot(k[:, sl].astype(np.float64)), v[:, sl]
        sc = qh @ kh.T / np.sqrt(hd)
        if causal:
            sc = np.where(np.tril(np.ones((S, S), bool)), sc, -np.inf)
        p = np.exp(sc - sc.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        out[:, sl] = p @ vh
    return out


def test_attention_prefill(oracle):
    """tools/p12_build_minicpm.py:770-781 composition vs float64 attention;
    causal row 0 equals v row 0 bitwise (a one-element softmax is exactly 1)."""
    rng = np.random.default_rng(11)
    S, H, hd = 40, 3, 64
    q, k, v = (rng.standard_normal((S, H * hd)).astype(np.float32) for _ in range(3))
    out = oracle.attention_prefill(q, k, v, H)
    ref = _attn_f64(q, k, v, H, 10000.0, True)
    rms = np.sqrt(np.mean(ref ** 2))
    assert np.abs(out - ref).max() <= 1e-5 * max(rms, 1)
    assert np.array_equal(out[0], v[0])
    nc = oracle.attention_prefill(q, k, v, H, causal=False)
    assert np.abs(nc - _attn_f64(q, k, v, H, 10000.0, False)).max() <= 1e-5 * max(rms, 1)


def test_attention_decode_matches_prefill(oracle):
    """tools/p13_kv_check.py strategy: decoding position S-1 against a cache
    of rotated K / raw V for 0..S-2 equals row S-1 of the full prefill."""
    rng = np.random.default_rng(12)
    S, H, hd, cap = 33, 2, 64, 48
    q, k, v = (rng.standard_normal((S, H * hd)).astype(np.float32) for _ in range(3))
    full = oracle.attention_prefill(q, k, v, H)
    kc = np.zeros((H, cap, hd), np.float32)
    vc = np.zeros((H, cap, hd), np.float32)
    for p in range(S - 1):
        oracle.attention_decode(q[p], k[p], v[p], kc, vc, p)
    out = oracle.attention_decode(q[S - 1], k[S - 1], v[S - 1], kc, vc, S - 1)
    assert np.abs(out - full[S - 1]).max() < 1e-5
    # the cache holds rotated K at each position
    for h in range(H):
        kr = oracle.rope(k[5, h * hd:(h + 1) * hd][None, :], 10000.0, 5)
        assert np.array_equal(kc[h, 5, :], kr[0])


# ---------------------------------------------------------------- decoder
def test_decoder_tiny_decode_equals_reprefill(oracle):
    """p13_kv_check strategy at the program level: the logits of a decode
    step equal the last-row logits of a prefill over the extended prompt;
    the greedy chain's first token is the argmax of the prefill logits."""
    from sparrow_amd import model as M
    cfg = M.tiny_config(n_layers=2, hidden=128, n_heads=2, inter=256, vocab=500)
    W = M.make_weights(cfg, seed=3)
    dec = oracle.DecoderOracle(W, cfg, cap=32)
    prompt = np.array([5, 17, 230, 499, 0, 42], np.int32)
    logits, _ = dec.prefill(prompt)
    t0 = int(np.argmax(logits))
    step_logits, _ = dec.step(t0, len(prompt))
    dec2 = oracle.DecoderOracle(W, cfg, cap=32)
    ext, _ = dec2.prefill(np.append(prompt, t0).astype(np.int32))
    rms = np.sqrt(np.mean(ext.astype(np.float64) ** 2))
    assert np.abs(step_logits - ext).max() <= 1e-4 * rms
    dec3 = oracle.DecoderOracle(W, cfg, cap=32)
    toks, margins = dec3.generate(prompt, 4)
    assert toks[0] == t0 and toks[1] == int(np.argmax(step_logits))
    assert np.all(margins >= 0)


# ------------------------------------------------- decoder, independent pin
def _f64_decoder_logits(W, cfg, tokens, variant=None):
    """float64 forward of the decoder program over `tokens`, written from the
    program text of tools/p12_build_minicpm.py:766-792 (layer) and :990-994
    (final norm and LM head), with OP_ROPE's rotation (core/src/interp.rs:
    1159-1223, angle pos * theta^(-2i/hd) in float64), OP_RMSNORM
    y = (x * inv) * g, the int8 GEMM C = (A . Q^T) * scale and causal
    softmax(scale * q.k) attention. It shares no code with the C oracle.
    Returns the logits of every row; row p is what a decode step at position
    p must give. `variant` plants one mistake for the can-fail controls."""
    H, NH, HD, eps = cfg["hidden"], cfg["n_heads"], cfg["head_dim"], cfg["eps"]
    S = len(tokens)
    f = np.float64

    def widen(t):
        return (t.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(f)

    def rmsnorm(x, g):
        inv = 1.0 / np.sqrt((x * x).mean(1, keepdims=True) + eps)
        return (x * inv) * g.astype(f)

    def q8(x, w, s):
        return (x @ w.astype(f).T) * s.astype(f)

    pos = np.arange(S, dtype=f)[:, None]
    inv_freq = f(cfg["theta"]) ** (-2.0 * np.arange(HD // 2, dtype=f) / HD)
    ang = pos * inv_freq
    co, si = np.cos(ang), np.sin(ang)

    def rope(x):
        x1, x2 = x[:, :HD // 2], x[:, HD // 2:]
        return np.concatenate([x1 * co - x2 * si, x1 * si + x2 * co], 1)

    causal = np.tril(np.ones((S, S), bool))
    h = widen(W["embed"][np.asarray(tokens)])
    for L in W["layers"]:
        in_ln, post_ln = (L["post_ln"], L["in_ln"]) if variant == "norms_swapped" else \
            (L["in_ln"], L["post_ln"])
        xn = rmsnorm(h, in_ln)
        q, k, v = q8(xn, L["wq"], L["sq"]), q8(xn, L["wk"], L["sk"]), q8(xn, L["wv"], L["sv"])
        att = np.empty_like(q)
        for hh in range(NH):
            cs = slice(hh * HD, (hh + 1) * HD)
            sc = rope(q[:, cs]) @ rope(k[:, cs]).T * f(cfg["attn_scale"])
            sc = np.where(causal, sc, -np.inf)
            p = np.exp(sc - sc.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            att[:, cs] = p @ v[:, cs]
        h2 = h + q8(att, L["wo"], L["so"])
        xn = rmsnorm(h2, post_ln)
        gate, up = q8(xn, L["wg"], L["sg"]), q8(xn, L["wu"], L["su"])
        if variant == "gate_up_swapped":
            gate, up = up, gate
        acts = gate / (1.0 + np.exp(-gate)) * up
        h = (h if variant == "residual_from_h" else h2) + q8(acts, L["wd"], L["sd"])
    xn = rmsnorm(h, W["final_norm"])
    return xn @ widen(W["lm_head"]).T


def test_decoder_oracle_vs_independent_f64(oracle):
    """Pins the C oracle's decoder composition (vo_decoder_prefill / step /
    generate) against the float64 forward above: the prefill's last-row
    logits and three greedy decode steps (each compared with the row of the
    float64 forward over the extended sequence) within 1e-5 * RMS, and the
    greedy tokens equal. Norm gains are random so a swapped norm shows.
    Controls: the same forward with gate and up swapped, the second
    residual taken from h instead of h2, or in_ln / post_ln swapped, is
    far outside the bound."""
    from sparrow_amd import model as M
    cfg = M.tiny_config(n_layers=2, hidden=128, n_heads=2, inter=256, vocab=500)
    W = M.make_weights(cfg, seed=5)
    rng = np.random.default_rng(55)
    for L in W["layers"]:
        L["in_ln"] = (1.0 + 0.5 * rng.standard_normal(cfg["hidden"])).astype(np.float32)
        L["post_ln"] = (1.0 + 0.5 * rng.standard_normal(cfg["hidden"])).astype(np.float32)
    W["final_norm"] = (1.0 + 0.5 * rng.standard_normal(cfg["hidden"])).astype(np.float32)
    prompt = np.array([3, 141, 59, 265, 358, 97, 9], np.int32)
    dec = oracle.DecoderOracle(W, cfg, cap=32)
    logits, _ = dec.prefill(prompt)

    def close(got, ref, tol=1e-5):
        return np.abs(got - ref).max() <= tol * np.sqrt(np.mean(ref ** 2))

    seq = list(prompt)
    ref = _f64_decoder_logits(W, cfg, seq)[-1]
    assert close(logits, ref)
    tok = int(np.argmax(logits))
    assert tok == int(np.argmax(ref))
    for step in range(3):
        step_logits, _ = dec.step(tok, len(seq))
        seq.append(tok)
        ref = _f64_decoder_logits(W, cfg, seq)[-1]
        assert close(step_logits, ref), step
        tok = int(np.argmax(step_logits))
        assert tok == int(np.argmax(ref))
    for variant in ("gate_up_swapped", "residual_from_h", "norms_swapped"):
        bad = _f64_decoder_logits(W, cfg, seq, variant)[-1]
        assert not close(step_logits, bad, tol=1e-2), variant


# ------------------------------------------- Backend primitives, jit helpers
def test_backend_dot_sum_oracle(oracle):
    """dot256 / sum256 (sys/src/x86_avx2/simd.rs:27-57, 380-405): float64
    within n * 2^-24 * sum|terms|; exact on small integers; n = 0 gives 0.
    Fold control: lane sums (l0+l4, l1+l5, l2+l6, l3+l7) = (2^24, 1, -2^24, 1)
    give 1 under hsum256's hadd order ((a+b)+(c+d)) and 2 under the hsum_ps
    order ((a+c)+(b+d)), so the restatement must return 1."""
    rng = np.random.default_rng(30)
    for n in (0, 1, 7, 8, 31, 32, 33, 1000, 4099):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        t = a.astype(np.float64) * b
        bound = (n + 1) * 2.0 ** -24 * np.abs(t).sum() + 1e-30
        assert abs(oracle.dot256(a, b) - t.sum()) <= bound
        assert abs(oracle.sum256(a) - a.astype(np.float64).sum()) <= \
            (n + 1) * 2.0 ** -24 * np.abs(a).sum() + 1e-30
        ia = rng.integers(-50, 50, n).astype(np.float32)
        ib = rng.integers(-50, 50, n).astype(np.float32)
        assert oracle.dot256(ia, ib) == float(ia.astype(np.int64) @ ib.astype(np.int64))
        assert oracle.sum256(ia) == float(ia.astype(np.int64).sum())
    lanes = np.float32([2 ** 24, 1, -2 ** 24, 1, 0, 0, 0, 0])
    assert oracle.dot256(lanes, np.ones(8, np.float32)) == 1.0
    assert oracle.sum256(lanes) == 1.0


def test_backend_max_oracle(oracle):
    """max256 (sys/src/x86_avx2/simd.rs:203-235): NaN-free input gives
    np.max; empty input -inf; MAXPS(a, b) returns b when a NaN is involved,
    so a NaN in lane 0 is dropped by the fold max(lane0, lane4) but a NaN in
    lane 4 survives it and is dropped one step later; an all-NaN block stays
    NaN and the tail's strict `>` never replaces it."""
    rng = np.random.default_rng(31)
    for n in (1, 5, 8, 9, 64, 1001):
        x = rng.standard_normal(n).astype(np.float32)
        assert oracle.max256(x) == x.max()
    assert oracle.max256(np.zeros(0, np.float32)) == -np.inf
    x = np.ones(8, np.float32)
    x[0] = np.nan
    assert oracle.max256(x) == 1.0
    x = np.ones(8, np.float32)
    x[4] = np.nan
    assert oracle.max256(x) == 1.0
    assert np.isnan(oracle.max256(np.full(9, np.nan, np.float32)))
    x = np.full(9, np.nan, np.float32)
    x[8] = 5.0
    assert np.isnan(oracle.max256(x))


def test_backend_elementwise_oracle(oracle):
    """axpy256 fuses a*x + y (one rounding) on the 8-blocks and rounds twice
    on the tail; add256 / scale_mul are single f32 operations (numpy float32
    is exact for them). The control a = x = 1 + 2^-12, y = -(1 + 2^-11):
    the fused result is 2^-24, the two-rounding one 0."""
    rng = np.random.default_rng(32)
    n = 45
    y = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    a = np.float32(0.37)
    got = oracle.axpy256(y, x, a)
    fused = (np.float64(a) * x + y).astype(np.float32)  # exact product, one rounding
    assert np.array_equal(got[:40], fused[:40])
    assert np.array_equal(got[40:], (a * x[40:] + y[40:]).astype(np.float32))
    e = np.float32(1 + 2 ** -12)
    yy = np.full(9, -(1 + 2 ** -11), np.float32)
    xx = np.full(9, e, np.float32)
    got = oracle.axpy256(yy, xx, e)
    assert np.all(got[:8] == np.float32(2 ** -24)) and got[8] == 0.0
    assert np.array_equal(oracle.add256(y, x), y + x)
    assert np.array_equal(oracle.scale_mul(x, a), a * x)


def test_layernorm_bias_outer_oracle(oracle):
    """layernorm (ops/src/kernels.rs:1308-1333) vs float64 within 1e-5; a
    constant row normalises to exactly b. jit_bias adds b to every row
    exactly. outer (:1416-1448) fuses on 8-blocks of j: the same control
    as axpy256 gives 2^-24 there and 0 on the tail."""
    rng = np.random.default_rng(33)
    x = rng.standard_normal((5, 77)).astype(np.float32)
    g = rng.standard_normal(77).astype(np.float32)
    b = rng.standard_normal(77).astype(np.float32)
    x[3] = 2.5
    y = oracle.layernorm(x, g, b, 1e-5)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-5) * g + b
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()
    assert np.array_equal(y[3], b)
    d = rng.standard_normal((4, 9)).astype(np.float32)
    assert np.array_equal(oracle.bias(d, b[:9]), d + b[:9])
    e = np.float32(1 + 2 ** -12)
    s = np.full((2, 10), -(1 + 2 ** -11), np.float32)
    out = oracle.outer(s, np.full(2, e, np.float32), np.full(10, e, np.float32))
    assert np.all(out[:, :8] == np.float32(2 ** -24)) and np.all(out[:, 8:] == 0.0)
    s = rng.standard_normal((3, 20)).astype(np.float32)
    v = rng.standard_normal(3).astype(np.float32)
    k = rng.standard_normal(20).astype(np.float32)
    out = oracle.outer(s, v, k, 0.5)
    vi = (v * np.float32(0.5)).astype(np.float32)
    assert np.array_equal(out[:, :16], (vi[:, None].astype(np.float64) * k[:16] + s[:, :16])
                          .astype(np.float32))
    assert np.array_equal(out[:, 16:], s[:, 16:] + vi[:, None] * k[16:])


# ------------------------------------------------------------ B1 backward
def _b1_case(seed, n=40, k0=11, d=None):
    rng = np.random.default_rng(seed)
    d = d or n
    w = rng.standard_normal((n, k0)).astype(np.float32)
    src = rng.integers(0, d, size=(n, k0)).astype(np.uint32)
    x = rng.standard_normal(d).astype(np.float32)
    dy = rng.standard_normal(n).astype(np.float32)
    return w, src, x, dy


def test_b1_backward_gradient_check(oracle):
    """b1_backward / b1_backward_dx (ops/src/b1_pure.rs:410, 642) are the
    gradients of L = sum_i dy_i * y_i with y_i = sum_j w_ij x[src_ij]:
    central differences of that forward (float64, a gather-sum, not the
    scatter under test) match dx and dw; a transposed scatter would not."""
    w, src, x, dy = _b1_case(50)
    n, k0 = w.shape

    def loss(xx, ww):
        return float((dy.astype(np.float64) * (ww.astype(np.float64) * xx[src]).sum(1)).sum())

    dx = oracle.b1_backward_dx(w, src, dy, np.zeros(n, np.float32))
    dw = oracle.b1_backward(w, src.astype(np.float32), dy, x)
    h = 1e-3
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    for s in range(n):
        e = np.zeros(n)
        e[s] = h
        fd = (loss(x64 + e, w64) - loss(x64 - e, w64)) / (2 * h)
        assert abs(fd - dx[s]) <= 1e-5 * (1 + abs(fd)), s
    for (i, j) in [(0, 0), (3, 7), (n - 1, k0 - 1), (17, 2)]:
        e = np.zeros((n, k0))
        e[i, j] = h
        fd = (loss(x64, w64 + e) - loss(x64, w64 - e)) / (2 * h)
        assert abs(fd - dw[i, j]) <= 1e-5 * (1 + abs(fd))


def test_b1_backward_fused_equals_separate(oracle):
    """ops/src/b1_pure.rs:466-490: the fused dw + dx pass is bit for bit the
    separate b1_backward (dw) and b1_backward_dx (dx), accumulating into
    non-zero buffers."""
    w, src, x, dy = _b1_case(51, n=64, k0=20)
    rng = np.random.default_rng(1)
    dw0 = rng.standard_normal(w.shape).astype(np.float32)
    dx0 = rng.standard_normal(64).astype(np.float32)
    dw, dx = oracle.b1_backward_fused(w, src, dy, x, dw0, dx0)
    assert np.array_equal(dw.view(np.uint32),
                          oracle.b1_backward(w, src.astype(np.float32), dy, x, dw0).view(np.uint32))
    assert np.array_equal(dx.view(np.uint32),
                          oracle.b1_backward_dx(w, src, dy, dx0).view(np.uint32))


def test_b1_backward_t8(oracle):
    """ops/src/kernels.rs:3229-3275 over source-major activations: dw is the
    token dot product (float64 within 1e-5), dxt[:, t] is token t's dx
    (float64 within 1e-5). Fold control: a connection whose eight lane sums
    are (2^24, 1, -2^24, 1, 0, 0, 0, 0) gets 1 (hsum256), not 2 (hsum_ps)."""
    w, src, _, _ = _b1_case(52, n=48, k0=9)
    rng = np.random.default_rng(2)
    t8 = 32
    xt = rng.standard_normal((48, t8)).astype(np.float32)
    dyt = rng.standard_normal((48, t8)).astype(np.float32)
    dxt, dw = oracle.b1_backward_t8(w, src, xt, dyt, np.zeros((48, t8), np.float32),
                                    np.zeros(w.shape, np.float32))
    ref_dw = (dyt.astype(np.float64)[:, None, :] * xt.astype(np.float64)[src]).sum(2)
    assert np.abs(dw - ref_dw).max() <= 1e-5 * np.abs(ref_dw).max()
    ref_dx = np.zeros((48, t8))
    np.add.at(ref_dx, src.ravel(), (dyt.astype(np.float64)[:, None, :] *
                                    w.astype(np.float64)[:, :, None]).reshape(-1, t8))
    assert np.abs(dxt - ref_dx).max() <= 1e-5 * np.abs(ref_dx).max()
    w1 = np.ones((1, 1), np.float32)
    s1 = np.zeros((1, 1), np.uint32)
    dyt1 = np.float32([[2 ** 24, 1, -2 ** 24, 1, 0, 0, 0, 0]])
    _, dw1 = oracle.b1_backward_t8(w1, s1, np.ones((1, 8), np.float32), dyt1,
                                   np.zeros((1, 8), np.float32), np.zeros((1, 1), np.float32))
    assert dw1[0, 0] == 1.0

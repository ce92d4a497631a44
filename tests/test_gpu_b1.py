"""B1 block-aligned sparse layer stack (8 layers, d=1536,
k0=32, 1024 tokens, tanh), bitwise against the oracle's t8 contract
(ops/src/kernels.rs:2163-2188) followed by tanh_f per layer."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_b1_stack_cfg4_bitwise(hip, oracle):
    from sparrow_amd import conn
    rng = np.random.default_rng(4)
    L, d, k0, T = 8, 1536, 32, 1024
    layers = [conn.make_block_aligned(rng, d, k0) for _ in range(L)]
    x = rng.standard_normal((T, d), dtype=np.float32)
    dev = [conn.DeviceConn(w, s, li) for li, (w, s) in enumerate(layers)]
    xb = conn.DeviceBuffer.from_array(x)
    yb = conn.DeviceBuffer(x.nbytes)
    conn.stack_forward(dev, xb.ptr, yb.ptr, T, act=4)
    y = yb.to_array((T, d), np.float32)
    for b in dev:
        b.free()
    xb.free()
    yb.free()
    # oracle: t8 contract + tanh_f per layer
    xt = oracle.transpose_t8(x, T)
    for w, s in layers:
        yt = oracle.b1_forward_t8(w, s, xt, T)
        xt = oracle.vmap("tanh", yt)
    ref = oracle.transpose_t8_back(xt, T)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_b1_stack_plan_equals_forward_and_replays(hip):
    """vmlm_b1_stack_create / run (the plan built once) give the bits of
    vmlm_b1_stack_forward at config 4; run captured into a HIP graph and
    replayed three times, with eager calls and syncs between the replays,
    equals the eager result every time; a stack beyond the one-kernel path
    returns 5."""
    import ctypes as C
    from sparrow_amd import VmlmError, check, conn, lib
    L = lib()
    rng = np.random.default_rng(44)
    d, k0, T = 1536, 32, 1024
    dev = [conn.DeviceConn(*conn.make_block_aligned(rng, d, k0), layer=li) for li in range(8)]
    x = rng.standard_normal((T, d), dtype=np.float32)
    xb = conn.DeviceBuffer.from_array(x)
    yf, yp, yg = (conn.DeviceBuffer(x.nbytes) for _ in range(3))
    conn.stack_forward(dev, xb.ptr, yf.ptr, T, act=4)
    plan = conn.StackPlan(dev)
    plan.run(xb.ptr, yp.ptr, T, act=4)
    ref = yf.to_array((T, d), np.float32)
    assert np.array_equal(yp.to_array((T, d), np.float32).view(np.uint32), ref.view(np.uint32))
    g = C.c_void_p()
    check(L.vmlm_hip_capture_begin(None))
    plan.run(xb.ptr, yg.ptr, T, act=4)
    check(L.vmlm_hip_capture_end(None, C.byref(g)))
    try:
        for _ in range(3):
            check(L.vmlm_hip_memset(yg.ptr, 0, x.nbytes))
            plan.run(xb.ptr, yp.ptr, T, act=4)
            check(L.vmlm_hip_sync())
            check(L.vmlm_hip_graph_launch(g, None))
            check(L.vmlm_hip_sync())
            assert np.array_equal(yg.to_array((T, d), np.float32).view(np.uint32),
                                  ref.view(np.uint32))
    finally:
        L.vmlm_hip_graph_destroy(g)
    plan.close()
    wide = [conn.DeviceConn(*conn.make_block_aligned(rng, 6000, 8))]
    with pytest.raises(VmlmError) as e:
        conn.StackPlan(wide)
    assert e.value.code == 5
    for b_ in dev + wide:
        b_.free()
    for b_ in (xb, yf, yp, yg):
        b_.free()


def test_b1_stack_prng_topology(hip, oracle):
    """The reference PRNG topology (core/src/conn_sparse.rs:157-214) as the
    index source, no activation."""
    from sparrow_amd import conn
    rng = np.random.default_rng(7)
    d, k0, T = 256, 20, 70
    src = conn.prng_sources(0, d, k0)
    assert src[0, 0] == oracle.neuron_conn_src(0, 0, 0, d, k0)
    assert all(src[i, j] == oracle.neuron_conn_src(0, i, j, d, k0)
               for i in (0, 1, 255) for j in range(k0))
    w = rng.standard_normal((d, k0), dtype=np.float32)
    x = rng.standard_normal((T, d), dtype=np.float32)
    dev = conn.DeviceConn(w, src)
    xb = conn.DeviceBuffer.from_array(x)
    yb = conn.DeviceBuffer(x.nbytes)
    conn.stack_forward([dev], xb.ptr, yb.ptr, T, act=0xFFFF)
    y = yb.to_array((T, d), np.float32)
    ref = oracle.transpose_t8_back(oracle.b1_forward_t8(w, src, oracle.transpose_t8(x, 72), T), T)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("d,k0s,T,act", [(1000, (32, 7, 1, 20), 37, 4),   # mixed k0, ragged
                                         (3000, (8, 8), 9, 0xFFFF),       # wide, no activation
                                         (40, (5,), 4, 4)])               # one pass, one block
def test_b1_stack_shapes(hip, oracle, d, k0s, T, act):
    """The one-kernel stack (plans padded to the widest layer with no-op
    steps, activations kept in LDS), bitwise against the oracle layer by
    layer."""
    from sparrow_amd import conn
    rng = np.random.default_rng(d + T)
    layers = [(rng.standard_normal((d, k0), dtype=np.float32),
               rng.integers(0, d, size=(d, k0)).astype(np.uint32)) for k0 in k0s]
    x = rng.standard_normal((T, d), dtype=np.float32)
    dev = [conn.DeviceConn(w, s, li) for li, (w, s) in enumerate(layers)]
    xb = conn.DeviceBuffer.from_array(x)
    yb = conn.DeviceBuffer(x.nbytes)
    conn.stack_forward(dev, xb.ptr, yb.ptr, T, act=act)
    y = yb.to_array((T, d), np.float32)
    for b in dev:
        b.free()
    xb.free()
    yb.free()
    xt = oracle.transpose_t8(x, (T + 7) // 8 * 8)
    for w, s in layers:
        xt = oracle.b1_forward_t8(w, s, xt, T)
        if act != 0xFFFF:
            xt = oracle.vmap("tanh", xt)
    ref = oracle.transpose_t8_back(xt, T)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------ B1 backward
def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.mark.parametrize("n,k0", [(200, 1), (200, 2), (96, 8), (200, 20), (64, 37), (1536, 32)])
def test_b1_backward_bitwise(hip, oracle, n, k0):
    """b1_backward (f32 ids), b1_backward_dx and the fused pass against the
    reference's scalar contract, bit for bit, accumulating into non-zero
    buffers; sources repeat (each source is read by ~k0 connections)."""
    from sparrow_amd import ops
    rng = np.random.default_rng(n + k0)
    w = rng.standard_normal((n, k0)).astype(np.float32)
    src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
    x = rng.standard_normal(n).astype(np.float32)
    dy = rng.standard_normal(n).astype(np.float32)
    dw0 = rng.standard_normal((n, k0)).astype(np.float32)
    dx0 = rng.standard_normal(n).astype(np.float32)
    dw, macs = ops.b1_backward(w, src, dy, x, dw0)
    assert macs == n * k0
    assert np.array_equal(bits(dw), bits(oracle.b1_backward(w, src.astype(np.float32), dy, x, dw0)))
    dx, accs = ops.b1_backward_dx(w, src, dy, dx0)
    assert accs == n * k0
    assert np.array_equal(bits(dx), bits(oracle.b1_backward_dx(w, src, dy, dx0)))
    fw, fx, _ = ops.b1_backward_fused(w, src, dy, x, dw0, dx0)
    ow, ox = oracle.b1_backward_fused(w, src, dy, x, dw0, dx0)
    assert np.array_equal(bits(fw), bits(ow)) and np.array_equal(bits(fx), bits(ox))


@pytest.mark.parametrize("n,k0,t8", [(96, 9, 32), (200, 20, 40), (1536, 32, 1024)])
def test_b1_backward_t8_bitwise(hip, oracle, n, k0, t8):
    """ops/src/kernels.rs:3229 over source-major activations: dw (eight FMA
    lanes folded in hsum256 order) and dxt (FMA per token, connections in
    order) bit for bit; the config-4 shape included."""
    from sparrow_amd import ops
    rng = np.random.default_rng(n * k0)
    w = (rng.standard_normal((n, k0)) / np.sqrt(k0)).astype(np.float32)
    src = rng.integers(0, n, size=(n, k0)).astype(np.uint32)
    xt = rng.standard_normal((n, t8)).astype(np.float32)
    dyt = rng.standard_normal((n, t8)).astype(np.float32)
    dxt0 = rng.standard_normal((n, t8)).astype(np.float32)
    dw0 = rng.standard_normal((n, k0)).astype(np.float32)
    gx, gw = ops.b1_backward_t8(w, src, xt, dyt, dxt0, dw0)
    ox, ow = oracle.b1_backward_t8(w, src, xt, dyt, dxt0, dw0)
    assert np.array_equal(bits(gw), bits(ow))
    assert np.array_equal(bits(gx), bits(ox))


def test_b1_backward_guards(hip):
    from sparrow_amd import VmlmError, ops
    w = np.ones((4, 2), np.float32)
    src = np.array([[0, 1], [2, 3], [1, 4], [0, 0]], np.uint32)  # 4 >= n
    with pytest.raises(VmlmError) as e:
        ops.b1_backward_fused(w, src, np.ones(4, np.float32), np.ones(4, np.float32))
    assert e.value.code == 9
    with pytest.raises(VmlmError) as e:
        ops.b1_backward_t8(w, np.zeros((4, 2), np.uint32), np.ones((4, 12), np.float32),
                           np.ones((4, 12), np.float32))
    assert e.value.code == 9  # t8 not a multiple of 8

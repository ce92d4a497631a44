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

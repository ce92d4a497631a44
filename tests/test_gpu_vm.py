"""GPU parity of the device-resident VM executor (vmlm_vm_*) against the
oracle's restatement of the reference VM (oracle.OracleVm), on the same
.vmb images.

Bars: the same exit codes and messages' subject for every guard; PRINT
output and slots bitwise where the op is elementwise, an index or a
selection (the p16 golden outputs, the op zoo's exact ops, greedy tokens);
f32-accumulated outputs (GEMMs, norms, attention, logits) within 1e-4 of
their RMS."""
import numpy as np
import pytest

import test_vm_oracle as T
from sparrow_amd import model as M
from sparrow_amd import programs, vmb

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gvm(hip):
    import sparrow_amd
    from sparrow_amd import vm
    sparrow_amd.init(0)
    return vm


def both(gvm, P, writes=(), reads=()):
    from oracle import oracle
    img = P.build()
    res = []
    with gvm.Vm(img) as g:
        for name, v in writes:
            g.write(name, v)
        g.run()
        res.append((g.output(), [g.read(r) for r in reads]))
    with oracle.OracleVm(img) as o:
        for name, v in writes:
            o.write(name, v)
        o.run()
        res.append((o.output(), [o.read(r) for r in reads]))
    return res


def codes(gvm, P):
    """The status (and message) of loading and running P on the GPU."""
    from sparrow_amd import VmlmError
    img = P.build()
    with pytest.raises(VmlmError) as e:
        g = gvm.Vm(img)
        try:
            g.run()
        finally:
            g.close()
    return e.value.code, str(e.value)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def test_vm_q8_kat_and_guards(gvm, oracle):
    (g, _), (o, _) = both(gvm, T.q8_program())
    assert np.array_equal(g, np.float32([-1, -1])) and np.array_equal(g, o)
    P = T.q8_program()
    x = P.act("x", 2, 4)
    P.text.insert(0, (vmb.OP["COPY"], 0, 0, x, P["w"], 0))
    assert codes(gvm, P)[0] == 9
    for prog, word in ((T.q8_program(scale=np.float32([0.5])), "shorter"),
                       (T.q8_program(fl=vmb.FL_TRANS_B), "NN"),
                       (T.q8_program(fl=vmb.FL_ACC), "acc"),
                       (T.q8_program(fl=vmb.FL_TRANS_B, dtype_w="bf16"), "bf16 NN")):
        c, m = codes(gvm, prog)
        assert c == 9 and word in m, m
    img = bytearray(T.q8_program().build())
    img[0] ^= 1
    from sparrow_amd import VmlmError
    with pytest.raises(VmlmError) as e:
        gvm.Vm(bytes(img))
    assert e.value.code == 3
    for op, code in ((43, 5), (67, 6)):
        P = T.q8_program()
        P.text.insert(0, (op, 0, 0, P["y"], P["y"], P["y"]))
        assert codes(gvm, P)[0] == code


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_vm_p16_compose_golden(gvm, oracle, k):
    (g, _), (o, _) = both(gvm, T.compose_program(k))
    want, nnz = T.P16_AFTER[k]
    assert np.array_equal(g[:4], np.float32(want)) and g[4] == nnz
    assert np.array_equal(bits(g), bits(o))


def test_vm_sparse_ungated_and_guards(gvm, oracle):
    (g, _), (o, _) = both(gvm, T.compose_program(0, gated=False, data="guards/"))
    assert np.array_equal(g, np.float32([50, 120, 0, 120, 4])) and np.array_equal(g, o)

    def bad(name):
        def tw(off, src, w, x):
            g = f"{T.GOLD}/p16_compose/guards/"
            return (np.fromfile(g + "offbad.bin", np.float32) if name == "off" else off,
                    np.fromfile(g + "srcbad.bin", np.float32) if name == "src" else src, w, x)
        return tw
    for name in ("off", "src"):
        assert codes(gvm, T.compose_program(0, False, data="guards/", tweak=bad(name)))[0] == 9
    for kv in (99, -1):
        P = vmb.Program()
        s = P.const("strc", np.fromfile(f"{T.GOLD}/p16_compose/guards/str.bin", np.float32)
                    .reshape(4, 1))
        kc = P.scalar("kc", float(kv))
        sel = P.act("sel", 4, 2)
        P.ins("TOPK_BY_STRENGTH", sel, s, kc)
        P.ins("HALT")
        assert codes(gvm, P)[0] == 9


def test_vm_topk_by_strength_random(gvm, oracle):
    """Segmented and flat selection on random strengths with ties, NaNs and
    signed zeros: the same selections and values, bitwise."""
    rng = np.random.default_rng(3)
    s = rng.integers(-4, 5, size=(37, 50)).astype(np.float32)
    s[3, 7] = np.nan
    s[5, 0] = np.nan
    s[9, :] = -0.0
    s[9, ::3] = 0.0
    P = vmb.Program()
    sc = P.const("sc", s)
    kc = P.scalar("kc", 9.0)
    sel = P.act("sel", 37, 24)
    P.ins("TOPK_BY_STRENGTH", sel, sc, kc, fl=vmb.FL_SELGATE)
    flat = P.const("flat", s[:20].reshape(1, -1))
    kf = P.scalar("kf", 150.0)
    fsel = P.act("fsel", 1000, 2)
    P.ins("TOPK_BY_STRENGTH", fsel, flat, kf)
    P.ins("HALT")
    (_, g), (_, o) = both(gvm, P, reads=("sel", "fsel"))
    for a, b in zip(g, o):
        assert np.array_equal(bits(a), bits(b))


def test_vm_op_zoo(gvm, oracle):
    """The elementwise, copy, selection and reduction opcodes against the
    oracle: bitwise except LN, BMM and the accumulating GEMMs (1e-4 RMS)."""
    rng = np.random.default_rng(5)
    P = vmb.Program()
    A = P.const("A", (rng.standard_normal((7, 20)) * 3).astype(np.float32))
    B = P.const("B", rng.standard_normal((7, 20)).astype(np.float32))
    col = P.const("col", rng.standard_normal((7, 1)).astype(np.float32))
    row = P.const("row", rng.standard_normal((1, 20)).astype(np.float32))
    one = P.scalar("one", 0.37)
    lohi = P.const("lohi", np.float32([[-1.5, 2.0]]))
    vec = P.const("vec", rng.standard_normal((20, 1)).astype(np.float32))
    g = P.const("g", rng.standard_normal((1, 20)).astype(np.float32))
    bb = P.const("bb", rng.standard_normal((1, 20)).astype(np.float32))
    Bm = P.const("Bm", rng.standard_normal((20, 9)).astype(np.float32))
    exact, approx = [], []
    for i, (op, b_, fl) in enumerate((("EXP", 0, 0), ("LOG", 0, 0), ("SIN", 0, 0), ("COS", 0, 0),
                                       ("NEG", 0, 0), ("GEMASK", 0, 0), ("CLAMP", lohi, 0),
                                       ("EWMAX", B, 0), ("EWADD", col, 0), ("EWMUL", row, 0),
                                       ("EWSUB", one, 0), ("EWDIV", B, 0), ("SCALE", one, 0),
                                       ("ACT", 0, 2), ("ACT", 0, 4), ("MASK_MUL", col, 0),
                                       ("SOFTMAX", 0, vmb.FL_CAUSAL), ("COPY", 0, 0))):
        d = P.act(f"d{i}", 7, 20)
        P.ins(op, d, A, b_, fl=fl)
        (approx if op == "SOFTMAX" else exact).append(f"d{i}")
    for name, op, shape, a_, b_ in (("t", "TRANSPOSE", (20, 7), A, 0), ("sm", "SUM", (7, 1), A, 0),
                                    ("mx", "MAX", (7, 1), A, 0), ("gv", "GEMV", (7, 1), A, vec),
                                    ("th", "TOPK_THRESH", (7, 1), A, 0),
                                    ("cc", "CONCAT", (7, 40), A, B),
                                    ("sl", "SLICE", (7, 5), A, 3)):
        d = P.act(name, *shape)
        P.ins(op, d, a_, b_, fl=3 if op == "TOPK_THRESH" else 0)
        (approx if op in ("GEMV",) else exact).append(name)
    ln = P.act("ln", 7, 20)
    P.ins("LN", ln, A, g, dt=bb)
    bm = P.act("bm", 7, 9)
    P.ins("BMM", bm, A, Bm)
    ou = P.act("ou", 7, 20)
    P.ins("COPY", ou, B)
    P.ins("OUTER", ou, col, row)
    bi = P.act("bi", 7, 20)
    P.ins("COPY", bi, A)
    P.ins("BIAS", bi, row)
    wc = P.act("wc", 7, 30)
    P.ins("WRITECOL", wc, A, 10)
    stk = P.act("stk", 3, 140)
    P.ins("PUSH", stk, A, 2)
    pp = P.act("pp", 7, 20)
    P.ins("POP", pp, stk, 2)
    exact += ["ou", "bi", "wc", "stk", "pp"]
    approx += ["ln", "bm"]
    P.ins("HALT")
    (_, g_), (_, o_) = both(gvm, P, reads=exact + approx)
    for name, a, b in zip(exact + approx, g_, o_):
        if name in exact:
            assert np.array_equal(bits(a), bits(b)), name
        else:
            rms = np.sqrt(np.mean(b.astype(np.float64) ** 2))
            assert np.abs(a - b).max() <= 1e-4 * rms, name


@pytest.mark.parametrize("m", [1, 3, 5, 20])
def test_vm_int8_gemm_swizzled_consts(gvm, oracle, m):
    """OP_GEMM over int8 constants: the 96-row weight is also held in the
    swizzled layout from load on (the small-row launch and the int8-row GEMM
    read it), the 100-row one stays row-major only. Both against the oracle
    VM within 1e-4 of each row's RMS, with the reference's non-finite
    pattern for a NaN row and a row holding +inf."""
    rng = np.random.default_rng(40 + m)
    k = 768
    P = vmb.Program()
    x = rng.standard_normal((m, k)).astype(np.float32)
    if m >= 3:
        x[1, 5] = np.nan
        x[2, 7] = np.inf
    X = P.const("x", x)
    outs = []
    for name, n in (("ws", 96), ("wr", 100)):
        w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        w[:8, 7] = 0
        W = P.const(name, w, "i8")
        sc = (np.abs(rng.normal(0, 0.02, n)) / 127 + 1e-6).astype(np.float32)
        S = P.const(name + "_sc", sc, rows=n, cols=1)
        Y = P.act("y" + name, m, n)
        P.ins("GEMM", Y, X, W, dt=S)
        outs.append("y" + name)
    P.ins("HALT")
    img = P.build()
    with gvm.Vm(img) as g:
        assert g.swizzled_consts() == 1
        g.run()
        got = [g.read(r) for r in outs]
    with oracle.OracleVm(img) as o:
        o.run()
        ref = [o.read(r) for r in outs]
    for a, b in zip(got, ref):
        for f in (np.isnan, np.isposinf, np.isneginf):
            assert np.array_equal(f(a), f(b)), f.__name__
        for i in range(m):
            if np.isfinite(b[i]).all():
                r = np.sqrt(np.mean(b[i].astype(np.float64) ** 2))
                assert np.abs(a[i] - b[i]).max() <= 1e-4 * r, i


@pytest.fixture(scope="module")
def tiny():
    cfg = M.tiny_config(n_layers=3, hidden=256, n_heads=4, inter=512, vocab=1000)
    return cfg, M.make_weights(cfg, seed=23)


def test_vm_decoder_program(gvm, oracle, tiny):
    """Prefill (p12 structure) and 5 unrolled greedy steps (p14 structure) on
    the GPU executor: every PRINTed logit row within 1e-4 of its RMS of the
    oracle VM's, and the same greedy tokens in st_gen."""
    cfg, W = tiny
    S, G, V = 9, 5, cfg["vocab"]
    prompt = M.make_prompts(cfg, 1, S, seed=4)[0]
    rl, _ = oracle.DecoderOracle(W, cfg, cap=S + G).prefill(prompt)
    P = programs.minicpm_program(cfg, W, S, G)
    (g, gg), (o, og) = both(gvm, P, writes=(("st_tok", prompt), ("st_gen", [np.argmax(rl)])),
                            reads=("st_gen",))
    assert np.array_equal(gg[0], og[0])
    g, o = g.reshape(-1, V), o.reshape(-1, V)
    for r in range(g.shape[0]):
        rms = np.sqrt(np.mean(o[r].astype(np.float64) ** 2))
        assert np.abs(g[r] - o[r]).max() <= 1e-4 * rms, r


def test_vm_looped_and_step_loop(gvm, tiny):
    """On the GPU: the LAYERB / LOOP_CNT prefill equals the unrolled one
    bitwise; the step-looped decode (runtime RoPE position, cache column and
    softmax width) gives the unrolled decode's greedy tokens."""
    cfg, W = tiny
    prompt = M.make_prompts(cfg, 1, 6, seed=8)[0]
    outs = []
    for looped in (False, True):
        with gvm.Vm(programs.minicpm_program(cfg, W, 6, looped=looped).build()) as g:
            g.write("st_tok", prompt)
            g.run()
            outs.append(g.output())
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    toks = []
    for step_loop in (False, True):
        with gvm.Vm(programs.minicpm_program(cfg, W, 6, 6, step_loop=step_loop).build()) as g:
            g.write("st_tok", prompt)
            g.write("st_gen", [11])
            g.run()
            toks.append(g.read("st_gen"))
    assert np.array_equal(toks[0], toks[1])


def test_vm_graph_segments_same_bits(gvm, tiny):
    """Loop bodies up to their first host opcode run eagerly on the first
    visit, are captured into a HIP graph on the second and replayed after.
    The step-looped decode (its body up to the PRINT of the logits) gives the
    same bits with graphs as without: every PRINTed value, the greedy chain,
    the caches and the scratch slots, over two runs of the same VM (the
    second replays from its first step, with the eager opcodes and
    synchronisations between replays). The LAYERB-looped prefill's layer body
    reads each layer's own scalars (eps, theta) on the host at a new layer
    base, which ends its capture: it runs opcode by opcode, with the same
    bits."""
    cfg, W = tiny
    nl, nh = cfg["n_layers"], cfg["n_heads"]
    prompt = M.make_prompts(cfg, 1, 6, seed=8)[0]
    slots = ["st_gen", "hdec", "xnd", "attd", "actsd"]
    slots += [f"st_kc{l}_{h}" for l in (0, nl - 1) for h in (0, nh - 1)]
    slots += [f"st_vc{l}_{h}" for l in (0, nl - 1) for h in (0, nh - 1)]
    img = programs.minicpm_program(cfg, W, 6, 7, step_loop=True, print_prefill=False).build()
    res = {}
    for on in (False, True):
        with gvm.Vm(img) as g:
            g.set_graphs(on)
            runs = []
            for _ in range(2):
                g.clear_output()
                g.write("st_tok", prompt)
                g.write("st_gen", [11])
                g.run()
                runs.append((g.output(), {r: g.read(r) for r in slots}))
            assert g.graph_segments() == (1 if on else 0)
        res[on] = runs
    for k in range(2):
        assert np.array_equal(bits(res[False][k][0]), bits(res[True][k][0])), k
        for r in slots:
            assert np.array_equal(bits(res[False][k][1][r]), bits(res[True][k][1][r])), (k, r)
    img = programs.minicpm_program(cfg, W, 6, looped=True).build()
    outs = {}
    for on in (False, True):
        with gvm.Vm(img) as g:
            g.set_graphs(on)
            g.write("st_tok", prompt)
            g.run()
            outs[on] = g.output()
            assert g.graph_segments() == 0
    assert np.array_equal(bits(outs[False]), bits(outs[True]))


@pytest.mark.parametrize("rewrite", [False, True])
def test_vm_graph_segment_constant_writes(gvm, oracle, rewrite):
    """A loop body whose ROPE angle comes from a constant scalar: captured
    after its first visit and replayed (one graph segment) when nothing
    writes the constant; when the body rewrites the constant (a COPY into
    it, which ends the segment before it and drops captured graphs), the
    body keeps running opcode by opcode. Either way the results equal the
    same VM without graphs and the oracle VM, bit for bit."""
    rng = np.random.default_rng(11)
    hd = 16

    def prog():
        P = vmb.Program()
        x0 = P.const("x0", rng_x)
        th = P.scalar("th", 10000.0)
        th2 = P.scalar("th2", 500.0)
        P.scalar("steps", 5.0)
        for name in ("x", "y", "acc", "cnt"):
            P.act(name, 1, hd if name != "cnt" else 1)
        P.ins("COPY", P["x"], x0)
        P.ins("COPY", P["cnt"], P["steps"])
        top = P.label()
        for i in range(10):
            P.ins("ROPE", P["y"], P["x"], th, dt=i)
            P.ins("EWADD", P["acc"], P["acc"], P["y"])
        if rewrite:
            P.ins("COPY", th, th2)
        P.ins("LOOP_CNT", top, P["cnt"])
        P.ins("HALT")
        return P

    rng_x = rng.standard_normal((1, hd)).astype(np.float32)
    img = prog().build()
    res = {}
    for on in (False, True):
        with gvm.Vm(img) as g:
            g.set_graphs(on)
            g.run()
            res[on] = g.read("acc")
            assert g.graph_segments() == (1 if on and not rewrite else 0)
    assert np.array_equal(bits(res[False]), bits(res[True]))
    with oracle.OracleVm(img) as o:
        o.run()
        assert np.array_equal(bits(o.read("acc")), bits(res[True]))


def test_vm_fused_head_runs(gvm, oracle, tiny):
    """The step-looped decode's per-head runs (cache append; attention) run
    as one launch each per layer: the same greedy tokens as the oracle VM,
    and the step logits, the last head's scratch slots, the K/V caches and
    the attention rows within 1e-4 RMS (they follow the projections' GEMM
    numerics; the runs' own rotation and copies are checked bitwise on exact
    inputs below). The unrolled program (compile-time positions) runs opcode
    by opcode."""
    cfg, W = tiny
    S, G = 6, 5
    prompt = M.make_prompts(cfg, 1, S, seed=9)[0]
    img = programs.minicpm_program(cfg, W, S, G, step_loop=True, print_prefill=False).build()
    nl, nh = cfg["n_layers"], cfg["n_heads"]
    exact = ["st_gen"]
    approx = ["kdh", "vdh", "kdrot", "kdT", "vdT", "qdh", "qdrot", "scd", "ctxd", "attd"]
    approx += [f"st_kc{l}_{h}" for l in (0, nl - 1) for h in (0, nh - 1)]
    approx += [f"st_vc{l}_{h}" for l in (0, nl - 1) for h in (0, nh - 1)]
    with gvm.Vm(img) as g:
        # per layer: the cache append with the attention, q/k/v, gate/up,
        # o and down each with its residual add, and the prompt's
        # column-by-column cache writes of every head
        assert g.fused_runs() == 5 * nl + nl * nh
        g.write("st_tok", prompt)
        g.write("st_gen", [11])
        g.run()
        gout, got = g.output(), {r: g.read(r) for r in exact + approx}
    with oracle.OracleVm(img) as o:
        o.write("st_tok", np.float32(prompt))
        o.write("st_gen", np.float32([11]))
        o.run()
        oout, ref = o.output(), {r: o.read(r) for r in exact + approx}
    for r in exact:
        assert np.array_equal(bits(got[r]), bits(ref[r])), r
    for r in approx:
        rms = np.sqrt(np.mean(ref[r].astype(np.float64) ** 2))
        assert np.abs(got[r] - ref[r]).max() <= 1e-4 * rms, r
    gl, ol = gout.reshape(G, -1), oout.reshape(G, -1)
    for s_ in range(G):
        rms = np.sqrt(np.mean(ol[s_].astype(np.float64) ** 2))
        assert np.abs(gl[s_] - ol[s_]).max() <= 1e-4 * rms, s_
    with gvm.Vm(programs.minicpm_program(cfg, W, S, G).build()) as g:
        # q/k/v, gate/up, o + add and down + add of every step, the prompt's
        # cache writes per head
        assert g.fused_runs() == 4 * nl * G + nl * nh


@pytest.mark.parametrize("m", [1, 3])
def test_vm_fused_gemm_runs(gvm, oracle, m):
    """q/k/v-like GEMMs of one input, and gate, up, ACT silu, EWMUL, at
    decode rows: one launch per run, the same bits as the same opcodes run
    one by one (a SHAPE between them breaks the runs) and within 1e-4 RMS of
    the oracle VM; a 100-row weight (row-major only) beside swizzled ones
    runs opcode by opcode."""
    rng = np.random.default_rng(70 + m)
    k = 768

    def prog(split, nq=96):
        P = vmb.Program()
        X = P.const("x", rng_x)
        outs = []
        for name, nrows in (("q", nq), ("k", 64), ("v", 64), ("gate", 128), ("up", 128)):
            W = P.const(name, ws[name][:nrows], "i8")
            S = P.const(name + "_sc", scs[name][:nrows], rows=nrows, cols=1)
            P.act("y" + name, m, nrows)
            outs.append(("y" + name, W, S))
        P.act("a", m, 128)
        for i, (y, W, S) in enumerate(outs):
            P.ins("GEMM", P[y], X, W, dt=S)
            if split:
                P.ins("SHAPE", 0, 0, 0)
        P.ins("ACT", P["a"], P["ygate"], fl=vmb.ACT["silu"])
        if split:
            P.ins("SHAPE", 0, 0, 0)
        P.ins("EWMUL", P["a"], P["a"], P["yup"])
        P.ins("HALT")
        return P

    rng_x = rng.standard_normal((m, k)).astype(np.float32)
    ws = {n: rng.integers(-127, 128, size=(128, k), dtype=np.int8)
          for n in ("q", "k", "v", "gate", "up")}
    scs = {n: (np.abs(rng.normal(0, 0.02, 128)) / 127 + 1e-6).astype(np.float32) for n in ws}
    names = ["yq", "yk", "yv", "ygate", "yup", "a"]
    res = {}
    for split in (False, True):
        img = prog(split).build()
        with gvm.Vm(img) as g:
            assert g.fused_runs() == (0 if split else 2)
            g.run()
            res[split] = {r: g.read(r) for r in names}
    with oracle.OracleVm(prog(False).build()) as o:
        o.run()
        ref = {r: o.read(r) for r in names}
    for r in names:
        assert np.array_equal(bits(res[False][r]), bits(res[True][r])), r
        rms = np.sqrt(np.mean(ref[r].astype(np.float64) ** 2))
        assert np.abs(res[False][r] - ref[r]).max() <= 1e-4 * rms, r
    img = prog(False, nq=100).build()
    with gvm.Vm(img) as g:
        g.run()
        y100 = g.read("yq")
    with oracle.OracleVm(img) as o:
        o.run()
        r100 = o.read("yq")
    rms = np.sqrt(np.mean(r100.astype(np.float64) ** 2))
    assert np.abs(y100 - r100).max() <= 1e-4 * rms


@pytest.mark.parametrize("hd,nh,C", [(8, 2, 6), (64, 3, 40)])
def test_vm_fused_runs_guard(gvm, hd, nh, C):
    """Fused runs over exact inputs (constant rows): the rotated and copied
    slots and the caches equal the oracle VM bitwise, the attention rows are
    within 1e-4 RMS. A fused run keeps its opcodes' device guards: a
    position past the cache (WRITECOL's runtime column) and a live width
    past the scores (SOFTMAX) trip the VM's guard (status 9), as opcode by
    opcode. At hd = 64 the append and the attention run as one launch, with
    the bits of the two runs launched apart (a SHAPE between them)."""
    rng = np.random.default_rng(2)
    xv = rng.standard_normal((1, nh * hd)).astype(np.float32)

    def prog(pos, live, split=False):
        P = vmb.Program()
        x = P.const("x", xv)
        th = P.scalar("theta", 10000.0)
        sc = P.scalar("sc", 0.5)
        pp = P.scalar("pos", float(pos))
        lv = P.scalar("live", float(live))
        for name, r, c in (("kh", 1, hd), ("vh", 1, hd), ("kr", 1, hd), ("kT", hd, 1),
                           ("vT", hd, 1), ("qh", 1, hd), ("qr", 1, hd), ("s", 1, C),
                           ("ctx", 1, hd), ("att", 1, nh * hd)):
            P.act(name, r, c)
        for h in range(nh):
            P.state(f"kc{h}", hd, C)
            P.state(f"vc{h}", hd, C)
        rt = vmb.FL_RUNTIME if hasattr(vmb, "FL_RUNTIME") else 64
        for h in range(nh):
            P.ins("SLICE", P["kh"], x, h * hd)
            P.ins("SLICE", P["vh"], x, h * hd)
            P.ins("ROPE", P["kr"], P["kh"], th, dt=pp, fl=rt)
            P.ins("TRANSPOSE", P["kT"], P["kr"])
            P.ins("TRANSPOSE", P["vT"], P["vh"])
            P.ins("WRITECOL", P[f"kc{h}"], P["kT"], 0, dt=pp, fl=rt)
            P.ins("WRITECOL", P[f"vc{h}"], P["vT"], 0, dt=pp, fl=rt)
        if split:
            P.ins("SHAPE", 0, 0, 0)
        for h in range(nh):
            P.ins("SLICE", P["qh"], x, h * hd)
            P.ins("ROPE", P["qr"], P["qh"], th, dt=pp, fl=rt)
            P.ins("GEMM", P["s"], P["qr"], P[f"kc{h}"], fl=vmb.FL_TRANS_B)
            P.ins("SCALE", P["s"], P["s"], sc)
            P.ins("SOFTMAX", P["s"], P["s"], lv, fl=rt)
            P.ins("GEMM", P["ctx"], P["s"], P[f"vc{h}"])
            P.ins("WRITECOL", P["att"], P["ctx"], h * hd)
        P.ins("HALT")
        return P

    from oracle import oracle as orc
    img = prog(2, 3).build()
    exact = ["kh", "vh", "kr", "kT", "vT", "qh", "qr", "kc0", "kc1", "vc0", "vc1"]
    with gvm.Vm(img) as g:
        assert g.fused_runs() == (1 if hd == 64 else 2)
        g.run()
        got = {r: g.read(r) for r in exact + ["att", "s", "ctx"]}
    if hd == 64:
        with gvm.Vm(prog(2, 3, split=True).build()) as g:
            assert g.fused_runs() == 2
            g.run()
            for r in exact + ["att", "s", "ctx"]:
                assert np.array_equal(bits(got[r]), bits(g.read(r))), r
    with orc.OracleVm(img) as o:
        o.run()
        ref = {r: o.read(r) for r in exact + ["att", "s", "ctx"]}
    for r in exact:
        assert np.array_equal(bits(got[r]), bits(ref[r])), r
    for r in ("att", "s", "ctx"):
        rms = np.sqrt(np.mean(ref[r].astype(np.float64) ** 2))
        assert np.abs(got[r] - ref[r]).max() <= 1e-4 * rms, r
    for pos, live in ((C, 3), (2, C + 1)):
        c, m = codes(gvm, prog(pos, live))
        assert c == 9 and "guard" in m, m


@pytest.mark.parametrize("m", [1, 3])
def test_vm_fused_gemm_add_runs(gvm, oracle, m):
    """An int8 GEMM at decode rows followed by the EWADD of its output and a
    residual (either operand order) runs as one launch whose epilogue also
    writes the sum: the GEMM output and the sum are the bits of the two
    opcodes run one by one (a SHAPE between them breaks the run), and match
    the oracle VM (GEMM within 1e-4 RMS)."""
    rng = np.random.default_rng(90 + m)
    k, nrows = 768, 128
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.integers(-127, 128, size=(nrows, k), dtype=np.int8)
    sc = (np.abs(rng.normal(0, 0.02, nrows)) / 127 + 1e-6).astype(np.float32)
    rv = rng.standard_normal((m, nrows)).astype(np.float32)

    def prog(split, swap):
        P = vmb.Program()
        X = P.const("x", x)
        W = P.const("w", w, "i8")
        S = P.const("w_sc", sc, rows=nrows, cols=1)
        R0 = P.const("r0", rv)
        for name in ("r", "y", "z"):
            P.act(name, m, nrows)
        P.ins("COPY", P["r"], R0)
        P.ins("GEMM", P["y"], X, W, dt=S)
        if split:
            P.ins("SHAPE", 0, 0, 0)
        if swap:
            P.ins("EWADD", P["z"], P["y"], P["r"])
        else:
            P.ins("EWADD", P["z"], P["r"], P["y"])
        P.ins("HALT")
        return P

    for swap in (False, True):
        res = {}
        for split in (False, True):
            with gvm.Vm(prog(split, swap).build()) as g:
                assert g.fused_runs() == (0 if split else 1)
                g.run()
                res[split] = {r: g.read(r) for r in ("y", "z")}
        for r in ("y", "z"):
            assert np.array_equal(bits(res[False][r]), bits(res[True][r])), (swap, r)
        with oracle.OracleVm(prog(False, swap).build()) as o:
            o.run()
            ref = {r: o.read(r) for r in ("y", "z")}
        for r in ("y", "z"):
            rms = np.sqrt(np.mean(ref[r].astype(np.float64) ** 2))
            assert np.abs(res[False][r] - ref[r]).max() <= 1e-4 * rms, (swap, r)
        assert np.array_equal(bits(res[False]["z"]), bits(rv + res[False]["y"]))


@pytest.mark.parametrize("k,inf", [(768, False), (2304, False), (2304, True)])
def test_vm_fused_norm_gemm_runs(gvm, oracle, k, inf):
    """An RMSNORM of one row followed by the GEMM run that reads it (q/k/v
    GEMMs; gate, up, ACT silu, EWMUL) runs as that run's one launch, which
    normalizes the row itself and also writes the RMSNORM's output: the
    normalized row and every output are the bits of the opcodes run one by
    one (a SHAPE after the RMSNORM keeps it out of the run), within 1e-4 RMS of the
    oracle VM. With an infinite input value the normalized row is NaN there
    and zero elsewhere, and every output NaN, as opcode by opcode."""
    rng = np.random.default_rng(110 + k)
    x = rng.standard_normal((1, k)).astype(np.float32) * 3
    if inf:
        x[0, 5] = np.inf
    gain = rng.uniform(0.5, 1.5, k).astype(np.float32)
    ws = {n: rng.integers(-127, 128, size=(128, k), dtype=np.int8)
          for n in ("q", "k", "v", "gate", "up")}
    scs = {n: (np.abs(rng.normal(0, 0.02, 128)) / 127 + 1e-6).astype(np.float32) for n in ws}

    def prog(split):
        P = vmb.Program()
        X = P.const("x", x)
        G = P.const("g", gain)
        E = P.scalar("eps", 1e-5)
        P.act("y", 1, k)
        P.act("y2", 1, k)
        outs = {}
        for name in ws:
            outs[name] = (P.const(name, ws[name], "i8"),
                          P.const(name + "_sc", scs[name], rows=128, cols=1))
            P.act("o" + name, 1, 128)
        P.act("a", 1, 128)
        P.ins("RMSNORM", P["y"], X, G, dt=E)
        if split:
            P.ins("SHAPE", 0, 0, 0)
        for name in ("q", "k", "v"):
            P.ins("GEMM", P["o" + name], P["y"], outs[name][0], dt=outs[name][1])
        P.ins("RMSNORM", P["y2"], X, G, dt=E)
        if split:
            P.ins("SHAPE", 0, 0, 0)
        for name in ("gate", "up"):
            P.ins("GEMM", P["o" + name], P["y2"], outs[name][0], dt=outs[name][1])
        P.ins("ACT", P["a"], P["ogate"], fl=vmb.ACT["silu"])
        P.ins("EWMUL", P["a"], P["a"], P["oup"])
        P.ins("HALT")
        return P

    names = ["y", "y2", "oq", "ok", "ov", "ogate", "oup", "a"]
    res = {}
    for split in (False, True):
        with gvm.Vm(prog(split).build()) as g:
            # the q/k/v and gate/up runs either way, with the RMSNORMs unsplit
            assert g.fused_runs() == 2
            assert g.fused_opcodes() == (7 if split else 9)
            g.run()
            res[split] = {r: g.read(r) for r in names}
    for r in names:
        assert np.array_equal(bits(res[False][r]), bits(res[True][r])), r
    if inf:  # inv = 1 / sqrt(inf) = 0: y is NaN at the infinity, +-0 elsewhere
        for r in ("y", "y2"):
            assert np.isnan(res[False][r][0, 5]) and np.all(res[False][r][0, 6:] == 0), r
        for r in names[2:]:
            assert np.all(np.isnan(res[False][r])), r
        return
    with oracle.OracleVm(prog(False).build()) as o:
        o.run()
        ref = {r: o.read(r) for r in names}
    for r in names:
        rms = np.sqrt(np.mean(ref[r].astype(np.float64) ** 2))
        assert np.abs(res[False][r] - ref[r]).max() <= 1e-4 * rms, r


@pytest.mark.parametrize("Q", [1, 2])
def test_vm_col_runs(gvm, oracle, Q):
    """Column-by-column writes (SLICE a column of x, WRITECOL it into y; one
    stream or two interleaved, as the decoder program caches its prompt's K
    and V) run as two strided copies per stream: y and the column slot equal
    the oracle VM bitwise. With a jump into the run, the part before the jump
    target runs opcode by opcode and the rest as a run, with the same result.
    A run whose last WRITECOL would pass y's width runs opcode by opcode and
    trips the same guard (status 9)."""
    rng = np.random.default_rng(4 + Q)
    R, S, Wd = 5, 7, 9

    def prog(yo=1, jump=False):
        P = vmb.Program()
        xs = [P.const(f"x{q}", rng.standard_normal((R, S)).astype(np.float32)) for q in range(Q)]
        for q in range(Q):
            P.act(f"c{q}", R, 1)
            P.state(f"y{q}", R, Wd)
        if jump:
            P.ins("JMP", 1 + 2 * Q)  # into the second column's pairs
        for p in range(S):
            for q in range(Q):
                P.ins("SLICE", P[f"c{q}"], xs[q], p)
                P.ins("WRITECOL", P[f"y{q}"], P[f"c{q}"], yo + p)
        P.ins("HALT")
        return P

    names = [f"{k}{q}" for q in range(Q) for k in ("c", "y")]
    for jump, runs in ((False, 1), (True, 1)):
        img = prog(jump=jump).build()
        with gvm.Vm(img) as g:
            assert g.fused_runs() == runs
            g.run()
            got = {r: g.read(r) for r in names}
        with oracle.OracleVm(img) as o:
            o.run()
            ref = {r: o.read(r) for r in names}
        for r in names:
            assert np.array_equal(bits(got[r]), bits(ref[r])), (jump, r)
    with gvm.Vm(prog(yo=Wd - S + 1).build()) as g:
        assert g.fused_runs() == 0
    c, m = codes(gvm, prog(yo=Wd - S + 1))
    assert c == 9 and "WRITECOL" in m, m


def test_vm_shared_const_pool(gvm, tiny):
    """Two VMs over the same mapped weights region share one device pool
    (one upload); both run and agree bitwise."""
    cfg, W = tiny
    P = programs.minicpm_program(cfg, W, 4)
    img = P.build()
    d = vmb.parse(img)
    weights = np.frombuffer(img[d["const_off"]:d["const_off"] + d["const_len"]], np.uint8).copy()
    before = gvm.pool_uploads()
    prompt = np.float32([1, 2, 3, 4])
    with gvm.Vm(img, weights) as a, gvm.Vm(img, weights) as b:
        assert gvm.pool_uploads() == before + 1
        for v in (a, b):
            v.write("st_tok", prompt)
            v.run()
        assert np.array_equal(bits(a.output()), bits(b.output()))


def _counter_program():
    """LOOP_CNT over a constant counter (3 rounds of acc += 1), then a SCALE
    by a constant factor before and after a COPY writes that factor."""
    P = vmb.Program()
    n = P.scalar("n", 3.0)
    one = P.scalar("one", 1.0)
    f = P.scalar("f", 2.0)
    x = P.const("x", np.float32([[1, 2, 3, 4]]))
    acc = P.act("acc", 1, 1)
    src = P.act("src", 1, 1)
    out = P.act("out", 1, 4)
    top = P.label()
    P.ins("EWADD", acc, acc, one)
    P.ins("LOOP_CNT", top, n)
    P.ins("SCALE", out, x, f)      # f read while it is 2
    P.ins("EWADD", src, acc, one)  # 4
    P.ins("COPY", f, src)          # the constant f becomes 4
    P.ins("SCALE", out, x, f)      # reads 4
    P.ins("PRINT", acc)
    P.ins("PRINT", out)
    P.ins("HALT")
    return P


def test_vm_constant_slot_writes(gvm, oracle):
    """A program may write constant slots (slot_mut makes no distinction,
    core/src/interp.rs:477): LOOP_CNT on a constant counter runs its body
    the counter's number of times, and a SCALE after a COPY into its constant
    factor uses the new value, as in the oracle. Over constants shared through
    mapped weights the write is refused with 9: the mapped pool is read-only
    (cpool_readonly, :87, 2357-2362)."""
    P = _counter_program()
    (g, _), (o, _) = both(gvm, P)
    assert np.array_equal(g, np.float32([3, 4, 8, 12, 16])) and np.array_equal(g, o)
    img = P.build()
    d = vmb.parse(img)
    weights = np.frombuffer(img[d["const_off"]:d["const_off"] + d["const_len"]], np.uint8).copy()
    from sparrow_amd import VmlmError
    with gvm.Vm(img, weights) as v:
        with pytest.raises(VmlmError) as e:
            v.run()
    assert e.value.code == 9 and "read-only" in str(e.value)


def test_vm_guard_flag_is_per_vm(gvm):
    """Each VM reports only its own device guards: a VM whose EMB row is out
    of range exits 9; another VM run afterwards, and one run while the
    library's own flag is raised by a device-API call, both succeed, and that
    flag is still there for its owner to read."""
    import ctypes as C

    from sparrow_amd import VmlmError, lib

    def emb_program(row):
        P = vmb.Program()
        t = P.const("t", np.arange(12, dtype=np.float32).reshape(4, 3))
        r = P.scalar("r", float(row))
        y = P.act("y", 1, 3)
        P.ins("EMB", y, t, r)
        P.ins("PRINT", y)
        P.ins("HALT")
        return P.build()

    with gvm.Vm(emb_program(99)) as bad, gvm.Vm(emb_program(2)) as good:
        with pytest.raises(VmlmError) as e:
            bad.run()
        assert e.value.code == 9
        good.run()
        assert np.array_equal(good.output(), np.float32([6, 7, 8]))
        L = lib()
        buf = [C.c_void_p() for _ in range(3)]
        for p, n in zip(buf, (8, 4, 12)):
            assert L.vmlm_hip_malloc(C.byref(p), n) == 0
        row = np.float32([7.0])  # a 2-row table
        assert L.vmlm_hip_memcpy_h2d(buf[1], row.ctypes.data, 4) == 0
        assert L.vmlm_hip_emb_bf16(buf[2], buf[0], 2, 2, buf[1], None) == 0
        assert L.vmlm_hip_sync() == 0
        good.clear_output()
        good.run()
        assert np.array_equal(good.output(), np.float32([6, 7, 8]))
        assert L.vmlm_hip_check_guards() == 9
        assert L.vmlm_hip_check_guards() == 0
        for p in buf:
            L.vmlm_hip_free(p)


def test_vm_row_kernels_past_one_grid(gvm):
    """Row-per-thread VM kernels cover every row when there are more rows
    than one launch's 65535 workgroups hold: SUM over 65535 x 256 + 1000 rows
    of one value (each row's sum is its value) and SPARSE_MATVEC over
    65535 x 64 + 1000 neurons of one connection each (y_j = w_j * x_j)."""
    rng = np.random.default_rng(9)
    n = 65535 * 256 + 1000
    P = vmb.Program()
    a = P.act("a", n, 1)
    s = P.act("s", n, 1)
    P.ins("SUM", s, a)
    P.ins("HALT")
    v = rng.standard_normal(n).astype(np.float32)
    with gvm.Vm(P.build()) as g:
        g.write("a", v)
        g.run()
        assert np.array_equal(bits(g.read("s").ravel()), bits(v))
    m = 65535 * 64 + 1000
    P = vmb.Program()
    off = P.act("off", m + 1, 1)
    src = P.act("src", m, 1)
    w = P.act("w", m, 1)
    x = P.act("x", m, 1)
    y = P.act("y", m, 1)
    P.ins("SPARSE_MATVEC", y, off, src, dt=x, fl=w)
    P.ins("HALT")
    wv = rng.standard_normal(m).astype(np.float32)
    xv = rng.standard_normal(m).astype(np.float32)
    with gvm.Vm(P.build()) as g:
        g.write("off", np.arange(m + 1, dtype=np.float32))
        g.write("src", np.arange(m, dtype=np.float32))
        g.write("w", wv)
        g.write("x", xv)
        g.run()
        assert np.array_equal(bits(g.read("y").ravel()), bits(wv * xv))

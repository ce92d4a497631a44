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

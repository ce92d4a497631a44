"""CPU checks of the .vmb writer (sparrow_amd.vmb), the program builder
(sparrow_amd.programs) and the oracle's restatement of the reference VM
(oracle/vmlm_vm_oracle.c), which is the checker of the GPU executor.

Pins: FNV-1a test vectors; the q8 KAT of tools/p13_q8_check.py on its
committed inputs and its negative cases (exit 9); the TOPK_BY_STRENGTH +
SPARSE_MATVEC outputs that examples/p16_compose/README.md prints for k = 1..4
on the committed inputs (bit-exact by the README's own account), a closed-form
ungated case and the guard cases (exit 9); and the decoder program against the
oracle's decoder (vo_decoder_*, itself pinned by the float64 forward in
test_oracle.py)."""
from pathlib import Path

import numpy as np
import pytest

from sparrow_amd import model as M
from sparrow_amd import programs, vmb

GOLD = str(Path(__file__).resolve().parent / "golden" / "reference")


def test_hash32_fnv1a_vectors():
    # published FNV-1a 32-bit vectors
    assert vmb.hash32("") == 0x811C9DC5
    assert vmb.hash32("a") == 0xE40C292C
    assert vmb.hash32("foobar") == 0xBF9CF968


def test_image_layout_roundtrip():
    P = vmb.Program()
    c = P.const("w", np.arange(6, dtype=np.float32).reshape(2, 3))
    x = P.act("x", 2, 3)
    s = P.state("s", 1, 5)
    P.ins("COPY", x, c)
    P.ins("HALT")
    img = P.build()
    d = vmb.parse(img)
    assert d["magic"] == vmb.MAGIC and d["version"] == 1
    assert d["text"][0] == (vmb.OP["COPY"], 0, 0, x, c, 0)
    assert d["consts"][0][:5] == (0, 24, 2, 3, vmb.DT_F32)
    assert d["slots"] == [(vmb.SLOT_CONST, 0, 2, 3), (vmb.SLOT_ACT, 0, 2, 3),
                          (vmb.SLOT_STATE, 0, 1, 5)]
    assert d["act_bytes"] == 64 and d["state_bytes"] == 64
    assert d["const_off"] == 32 + 32 and d["const_len"] == 64


def q8_program(scale=None, fl=0, dtype_w="i8"):
    P = vmb.Program()
    a = P.const("a", np.fromfile(f"{GOLD}/q8_a.f32", np.float32).reshape(1, 4))
    wq = np.fromfile(f"{GOLD}/q8_w.i8", np.int8).reshape(2, 4)
    if dtype_w == "bf16":
        wq = (wq.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    w = P.const("w", wq, dtype_w)
    sc = np.fromfile(f"{GOLD}/q8_scale.f32", np.float32).reshape(2, 1) if scale is None else scale
    s = P.const("sc", sc, rows=sc.size, cols=1)
    y = P.act("y", 1, 2)
    P.ins("GEMM", y, a, w, dt=s, fl=fl)
    P.ins("PRINT", y)
    P.ins("HALT")
    return P


def run_oracle(img):
    from oracle import oracle
    with oracle.OracleVm(img) as vm:
        vm.run()
        return vm.output()


def expect_exit(img, code, where="run"):
    from oracle import oracle
    if where == "load":
        with pytest.raises(oracle.VmError) as e:
            oracle.OracleVm(img)
    else:
        with oracle.OracleVm(img) as vm, pytest.raises(oracle.VmError) as e:
            vm.run()
    assert e.value.code == code, e.value.msg
    return e.value.msg


def test_vm_q8_kat_and_guards(oracle):
    """tools/p13_q8_check.py: GEMM with an int8 B and its scale slot gives
    [[-1, -1]]; an int8 const read by COPY is refused at load, a scale
    shorter than N rows, an NN or accumulating int8 GEMM and a bf16 NN GEMM
    are refused when they run (all exit 9)."""
    assert np.array_equal(run_oracle(q8_program().build()), np.float32([-1, -1]))
    P = q8_program()
    x = P.act("x", 2, 4)
    P.text.insert(0, (vmb.OP["COPY"], 0, 0, x, P["w"], 0))
    assert "i8" in expect_exit(P.build(), 9, "load")
    assert "shorter" in expect_exit(q8_program(scale=np.float32([0.5])).build(), 9)
    assert "NN" in expect_exit(q8_program(fl=vmb.FL_TRANS_B).build(), 9)
    assert "acc" in expect_exit(q8_program(fl=vmb.FL_ACC).build(), 9)
    bf = q8_program(fl=vmb.FL_TRANS_B, dtype_w="bf16")
    assert "bf16 NN" in expect_exit(bf.build(), 9)


def test_vm_load_and_op_codes(oracle):
    """Bad magic exits 3, an unknown const dtype 9 at load, an unimplemented
    opcode 5 and a training opcode 6 (core/src/interp.rs:2346-2376)."""
    img = bytearray(q8_program().build())
    img[0] ^= 1
    expect_exit(bytes(img), 3, "load")
    P = q8_program()
    P.consts[0].dtype = 9
    expect_exit(P.build(), 9, "load")
    for op, code in ((43, 5), (67, 6)):
        P = q8_program()
        P.text.insert(0, (op, 0, 0, P["y"], P["y"], P["y"]))
        expect_exit(P.build(), code)


def compose_program(k, gated=True, nnz=True, data="", tweak=None):
    """TOPK_BY_STRENGTH (segmented) feeding SPARSE_MATVEC (selgate) over the
    committed CSR of examples/p16_compose; the selection slot must follow
    the src slot (the reference's src + 1 convention)."""
    g = f"{GOLD}/p16_compose/{data}"
    off = np.fromfile(g + "off.bin", np.float32)
    src = np.fromfile(g + "src.bin", np.float32)
    w = np.fromfile(g + "w.bin", np.float32)
    x = np.fromfile(g + "x.bin", np.float32)
    n, nnz_ = off.size - 1, src.size
    m = nnz_ // n
    if tweak:
        off, src, w, x = tweak(off, src, w, x)
    P = vmb.Program()
    offc = P.const("offc", off.reshape(-1, 1))
    srcc = P.const("srcc", src.reshape(-1, 1))
    wvc = P.const("wvc", w.reshape(-1, 1))
    xvc = P.const("xvc", x.reshape(-1, 1))
    kc = P.scalar("kc", float(k))
    so = P.act("off", off.size, 1)
    si = P.act("srci", src.size, 1)
    sel = P.act("sel", n, 2 * max(int(k), 1) if gated else 2)
    wv = P.act("wv", w.size, 1)
    xv = P.act("xv", x.size, 1)
    kk = P.act("kk", 1, 1)
    y = P.act("y", n + 1, 1)
    assert sel == si + 1
    for d, c in ((so, offc), (si, srcc), (wv, wvc), (xv, xvc), (kk, kc)):
        P.ins("COPY", d, c)
    if gated:
        st = P.const("str2c", np.fromfile(f"{GOLD}/p16_compose/str2d.bin", np.float32)
                     .reshape(n, m))
        sstr = P.act("str", n, m)
        P.ins("COPY", sstr, st)
        P.ins("TOPK_BY_STRENGTH", sel, sstr, kk, fl=vmb.FL_SELGATE)
    fl = (wv & vmb.SPARSE_WSLOT_MASK) | (vmb.FL_NNZ if nnz else 0) | \
        (vmb.FL_SELGATE if gated else 0)
    P.ins("SPARSE_MATVEC", y, so, si, dt=xv, fl=fl)
    P.ins("PRINT", y)
    P.ins("HALT")
    return P


# examples/p16_compose/README.md, "AFTER -- same x, same CSR, k varied"
P16_AFTER = {1: ([1.34999990, 1.80000007, 2.09999990, 1.50000000], 4.0),
             2: ([1.49999988, 2.80000019, 3.50000000, 1.92499995], 8.0),
             3: ([1.44999993, 3.10000014, 4.84999990, 1.72499990], 12.0),
             4: ([1.22499990, 3.02500010, 5.65000010, 1.27499986], 16.0)}


@pytest.mark.parametrize("k", [1, 2, 3, 4])
def test_vm_p16_compose_golden(oracle, k):
    y = run_oracle(compose_program(k).build())
    want, nnz = P16_AFTER[k]
    assert np.array_equal(y[:4], np.float32(want)), (y, want)
    assert y[4] == nnz


def test_vm_sparse_ungated_and_guards(oracle):
    """Ungated SPARSE_MATVEC on the guard fixtures: y = sum of w * x[src] per
    CSR row, first term assigned (closed form), nnz = 4. Guards (exit 9): k
    above L, negative k, an offset past nnz, a source id past x."""
    y = run_oracle(compose_program(0, gated=False, data="guards/").build())
    assert np.array_equal(y, np.float32([1 * 10 + 2 * 20, 3 * 40, 0, 4 * 30, 4]))

    def bad(name):
        def tw(off, src, w, x):
            g = f"{GOLD}/p16_compose/guards/"
            if name == "off":
                off = np.fromfile(g + "offbad.bin", np.float32)
            if name == "src":
                src = np.fromfile(g + "srcbad.bin", np.float32)
            return off, src, w, x
        return tw
    assert "offsets" in expect_exit(compose_program(0, False, data="guards/",
                                                    tweak=bad("off")).build(), 9)
    assert "src_id" in expect_exit(compose_program(0, False, data="guards/",
                                                   tweak=bad("src")).build(), 9)
    for kv in (99, -1):
        P = vmb.Program()
        s = P.const("strc", np.fromfile(f"{GOLD}/p16_compose/guards/str.bin", np.float32)
                    .reshape(4, 1))
        kc = P.scalar("kc", float(kv))
        sel = P.act("sel", 4, 2)
        P.ins("TOPK_BY_STRENGTH", sel, s, kc)
        P.ins("HALT")
        expect_exit(P.build(), 9)


@pytest.fixture(scope="module")
def tiny():
    cfg = M.tiny_config(n_layers=2, hidden=128, n_heads=2, inter=256, vocab=300)
    return cfg, M.make_weights(cfg, seed=21)


def run_program(P, prompt, first=None):
    from oracle import oracle
    with oracle.OracleVm(P.build()) as vm:
        vm.write("st_tok", np.float32(prompt))
        if first is not None:
            vm.write("st_gen", np.float32([first]))
        vm.run()
        out = vm.output()
        gen = vm.read("st_gen")[0] if first is not None else None
    return out, gen


def test_vm_decoder_program_matches_decoder_oracle(oracle, tiny):
    """The prefill program (p12 structure) gives the oracle decoder's
    last-row logits bit for bit; three unrolled greedy steps (p14
    structure, in-program argmax fed back through st_gen) give its chain and
    its step logits bit for bit."""
    cfg, W = tiny
    S, G, V = 6, 3, cfg["vocab"]
    prompt = np.array([5, 77, 123, 250, 9, 42], np.int32)
    ref = oracle.DecoderOracle(W, cfg, cap=S + G)
    rl, _ = ref.prefill(prompt)
    out, _ = run_program(programs.minicpm_program(cfg, W, S), prompt)
    assert np.array_equal(out.reshape(S, V)[-1].view(np.uint32), rl.view(np.uint32))
    t0 = int(np.argmax(rl))
    out, gen = run_program(programs.minicpm_program(cfg, W, S, G), prompt, first=t0)
    steps = out[S * V:].reshape(G, V)
    toks = [t0]
    for s in range(G):
        sl, _ = ref.step(toks[-1], S + s)
        assert np.array_equal(steps[s].view(np.uint32), sl.view(np.uint32)), s
        toks.append(int(np.argmax(sl)))
    assert np.array_equal(gen, np.float32(toks))


def test_vm_looped_layers_equal_unrolled(oracle, tiny):
    """LAYERB + LOOP_CNT over one layer template (p12 --loop) gives the
    unrolled prefill's logits bit for bit, and the base is restored after
    the loop (final_norm and the LM head are read at their own offsets)."""
    cfg, W = tiny
    prompt = np.array([1, 2, 3, 299, 150], np.int32)
    a, _ = run_program(programs.minicpm_program(cfg, W, 5), prompt)
    b, _ = run_program(programs.minicpm_program(cfg, W, 5, looped=True), prompt)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_vm_step_loop_equals_unrolled(oracle, tiny):
    """One decode step as a LOOP_CNT body with the RoPE position, cache
    column and softmax width read from slots: the same greedy chain as the
    unrolled program and step logits within 1e-6 of their RMS (the scores
    and context run over the whole cache width, zeros past the live
    positions)."""
    cfg, W = tiny
    S, G, V = 4, 4, cfg["vocab"]
    prompt = np.array([17, 3, 260, 99], np.int32)
    a, ga = run_program(programs.minicpm_program(cfg, W, S, G), prompt, first=7)
    b, gb = run_program(programs.minicpm_program(cfg, W, S, G, step_loop=True), prompt,
                        first=7)
    assert np.array_equal(ga, gb)
    la, lb = a[S * V:].reshape(G, V), b[S * V:].reshape(G, V)
    for s in range(G):
        rms = np.sqrt(np.mean(la[s].astype(np.float64) ** 2))
        assert np.abs(la[s] - lb[s]).max() <= 1e-6 * rms, s

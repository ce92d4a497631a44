"""The reference's P16 sparse-op programs on both VMs: the flat
TOPK_BY_STRENGTH -> SPARSE_MATVEC layer of examples/p16_ops (README.md:32-48)
on its committed inputs (tests/golden/reference/p16_ops/*.bin, byte-identical
to examples/p16_ops/w/*.bin), and the guard programs of
examples/p16_ops/guards/*.vml and examples/p16_compose/guards/*.vml with the
messages tools/p16_guardprobe.py expects (README.md:59-74).

Each program is rebuilt here with sparrow_amd.vmb from a case table (slot
shapes, constants, instructions); no .vml text is kept. The oracle VM runs
on the CPU; the same images run on the GPU executor in the `gpu` tests."""
import numpy as np
import pytest

from sparrow_amd import vmb

from test_vm_oracle import GOLD

OPS = f"{GOLD}/p16_ops"
GUARD = f"{GOLD}/p16_compose/guards"  # = examples/p16_ops/guards/w (same bytes)
COMPOSE = f"{GOLD}/p16_compose"


def f32(path):
    return np.fromfile(path, np.float32)


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# ----------------------------------------------------------------- the layer
def layer_program(off="off", src="src", w="w", st="str", k="k"):
    """examples/p16_ops/p16_layer.vml: 6 inputs, 4 neurons, CSR of the kept
    connections; TOPK_BY_STRENGTH over the 7 strengths (flat: sel [L,2]),
    then SPARSE_MATVEC with the performed-term count (FL_NNZ) in y[4]."""
    o, s, wv, sv = f32(f"{OPS}/{off}.bin"), f32(f"{OPS}/{src}.bin"), f32(f"{OPS}/{w}.bin"), \
        f32(f"{OPS}/{st}.bin")
    x, kv = f32(f"{OPS}/x.bin"), f32(f"{OPS}/{k}.bin")
    n, L = o.size - 1, s.size
    P = vmb.Program()
    c = [P.const(nm, a.reshape(-1, 1)) for nm, a in
         (("offc", o), ("srcc", s), ("wvc", wv), ("xvc", x), ("kc", kv), ("strc", sv))]
    so = P.act("off", n + 1, 1)
    si = P.act("srci", L, 1)
    swv = P.act("wv", L, 1)
    sx = P.act("xv", x.size, 1)
    sst = P.act("str", L, 1)
    sk = P.act("kk", 1, 1)
    sel = P.act("sel", L, 2)
    y = P.act("y", n + 1, 1)
    for d, cc in zip((so, si, swv, sx, sk, sst), c):
        P.ins("COPY", d, cc)
    P.ins("TOPK_BY_STRENGTH", sel, sst, sk)
    P.ins("SPARSE_MATVEC", y, so, si, dt=sx, fl=vmb.sparse_matvec_fl(swv, nnz=True))
    P.ins("HALT")
    return P


# examples/p16_ops/README.md:32-39: engine y (bit-exact with Python), nnz = 7
P16_Y = np.float32([0.14999985694885254, -2.700000047683716, 2.0999999046325684,
                    -3.174999952316284])


def flat_topk(strengths, k):
    """The flat selection rule stated in examples/p16_ops/README.md (rows of
    dst: surviving index ascending, its strength; rows nk.. zero) computed
    by brute force for finite strengths: the k largest values, a lower index
    first among equal ones."""
    order = sorted(range(strengths.size), key=lambda i: (-float(strengths[i]), i))
    keep = sorted(order[:k])
    out = np.zeros((strengths.size, 2), np.float32)
    for r, i in enumerate(keep):
        out[r] = (i, strengths[i])
    return out


def check_layer(run):
    """run(program, reads) -> (output, [slot values]) on one VM."""
    _, (y, sel) = run(layer_program(), ("y", "sel"))
    y = y.ravel()
    assert np.array_equal(bits(y[:4]), bits(P16_Y)) and y[4] == 7.0
    assert np.array_equal(bits(sel), bits(flat_topk(f32(f"{OPS}/str.bin"), 2)))
    assert sel[:2, 0].tolist() == [0.0, 4.0]  # ascending (the D4 control)
    # the dense-as-CSR control: every (j, i) pair kept, the count reads 24
    _, (y, sel) = run(layer_program("dense_off", "dense_src", "dense_w", "dense_str"),
                      ("y", "sel"))
    y = y.ravel()
    W = f32(f"{OPS}/dense_w.bin").reshape(4, 6).astype(np.float64)
    dense = W @ f32(f"{OPS}/x.bin").astype(np.float64)
    assert y[4] == 24.0 and np.abs(y[:4] - dense).max() <= 1e-6 * np.abs(dense).max()
    assert np.array_equal(bits(sel), bits(flat_topk(f32(f"{OPS}/dense_str.bin"), 2)))
    # the thinner CSR (one kept connection per neuron, k = 1)
    _, (y, sel) = run(layer_program("off_k1", "src_k1", "w_k1", "str_k1", "k1"), ("y", "sel"))
    x = f32(f"{OPS}/x.bin")
    want = f32(f"{OPS}/w_k1.bin") * x[f32(f"{OPS}/src_k1.bin").astype(int)]
    assert np.array_equal(bits(y.ravel()[:4]), bits(want)) and y.ravel()[4] == 4.0
    assert np.array_equal(bits(sel), bits(flat_topk(f32(f"{OPS}/str_k1.bin"), 1)))


def test_flat_topk_rule_brute_force():
    """The brute-force rule itself on a hand-checked case and a tie."""
    s = np.float32([1.35, -1.2, -1.8, -0.9, 2.1, 0.425, -3.6])
    assert flat_topk(s, 2)[:2, 0].tolist() == [0.0, 4.0]
    assert flat_topk(np.float32([1, 3, 3, 2]), 2)[:2, 0].tolist() == [1.0, 2.0]
    assert flat_topk(np.float32([1, 3, 3, 2]), 1)[:1, 0].tolist() == [1.0]


def oracle_run(P, reads=()):
    from oracle import oracle
    with oracle.OracleVm(P.build()) as o:
        o.run()
        return o.output(), [o.read(r) for r in reads]


def test_p16_layer_oracle(oracle):
    check_layer(oracle_run)


# ----------------------------------------------------------------- guards
def guard_program(case):
    """One guard program of tools/p16_guardprobe.py / examples/p16_*/guards,
    described by `case`: slot shape overrides, constant file overrides, and
    the final instruction(s)."""
    shapes = dict(case.get("shapes", {}))
    gate = case.get("gate", False)
    data = case.get("data", GUARD)
    files = dict(offc="off", srcc="src", wvc="w", xvc="x", k2c="k2", strc="str")
    files.update(case.get("files", {}))
    base = {"off": (5, 1), "srci": (4, 1), "wv": (4, 1), "xv": (4, 1), "str": (4, 1),
            "kk": (1, 1), "sel": (4, 2), "y": (5, 1)}
    order = ["off", "srci", "wv", "xv", "str", "kk", "sel", "y"]
    if gate:  # selgate layout: sel right after srci (the src + 1 convention)
        base.update(sel=(4, 8), str=(4, 4))
        order = ["off", "srci", "sel", "wv", "xv", "str", "kk", "y"]
    if data == COMPOSE:
        files = dict(offc="off", srcc="src", wvc="w", xvc="x", k2c="k2", strc="str2d")
        base.update(srci=(24, 1), wv=(24, 1), xv=(6, 1), str=(4, 6))
    base.update(shapes)
    P = vmb.Program()
    const = {}
    for name, fn in files.items():
        a = f32(f"{data}/{fn}.bin")
        const[name] = P.const(name, a.reshape(4, 6) if fn == "str2d" else a.reshape(-1, 1))
    for extra, fn in case.get("extra_consts", {}).items():
        const[extra] = P.const(extra, f32(f"{data}/{fn}.bin").reshape(-1, 1))
    S = {}
    for nm in order:
        if nm in base and base[nm] is not None:
            S[nm] = P.act(nm, *base[nm])
    S["zz"] = P.act("zz", 0, 0)   # names used but never shaped: width 0
    S["zo"] = P.act("zo", 0, 0)
    copies = [("off", "offc"), ("srci", "srcc"), ("wv", "wvc"), ("xv", "xvc"), ("kk", "k2c"),
              ("str", "strc")]
    for d, c in copies:
        if d in S and d not in case.get("no_copy", ()):
            P.ins("COPY", S[d], const[c])
    for op in case["ops"]:
        kind, *args = op
        if kind == "topk":
            dst, src, k, seg = args
            P.ins("TOPK_BY_STRENGTH", S[dst], S[src], const.get(k, S.get(k)),
                  fl=vmb.FL_SELGATE if seg else 0)
        else:
            dst, off, src, w, x, nnz, sg = args
            P.ins("SPARSE_MATVEC", S[dst], S[off], S[src], dt=S[x],
                  fl=vmb.sparse_matvec_fl(S[w], nnz=nnz, selgate=sg))
    if case.get("print"):
        P.ins("PRINT", S["y"])
    P.ins("HALT")
    return P


def spmv(dst="y", off="off", x="xv", nnz=True, sg=False):
    return ("spmv", dst, off, "srci", "wv", x, nnz, sg)


SPMV = spmv()
GATED = spmv(sg=True)
GUARDS = {
    # examples/p16_ops/guards (tools/p16_guardprobe.py), message substrings
    "k___L": (dict(ops=[("topk", "sel", "str", "k99c", False)],
                   extra_consts={"k99c": "k99"}), "k > L"),
    "k_negative": (dict(ops=[("topk", "sel", "str", "knegc", False)],
                        extra_consts={"knegc": "kneg"}), "negative or NaN"),
    "src_slot_zero_width": (dict(ops=[("topk", "sel", "zz", "k2c", False)]), "width 0"),
    "dst_not__L_2": (dict(shapes={"sel": (4, 1)}, ops=[("topk", "sel", "str", "k2c", False)]),
                     "dst must be [L,2]"),
    "dst_rows___L": (dict(shapes={"sel": (2, 2)}, ops=[("topk", "sel", "str", "k2c", False)]),
                     "dst needs L rows"),
    "selgate__odd_sel_width": (dict(gate=True, shapes={"sel": (4, 7)},
                                    ops=[GATED]),
                               "selgate needs an even sel width"),
    "selgate__sel_rows___n_neurons": (dict(gate=True, shapes={"sel": (2, 8)},
                                           ops=[GATED]), "sel table too small"),
    "selgate__TOPK_k___segment_width": (dict(gate=True, shapes={"sel": (4, 2)},
                                             ops=[("topk", "sel", "str", "k2c", True)]),
                                        "k > dst segment width"),
    "selgate__TOPK_segmented_dst_rows____src_rows": (
        dict(gate=True, shapes={"sel": (3, 8)}, ops=[("topk", "sel", "str", "k2c", True)]),
        "segmented dst rows != src rows"),
    "selgate__sel_index_outside_its_CSR_row": (
        dict(gate=True, files={"offc": "off_tiny", "strc": "str_tiny"},
             ops=[("topk", "sel", "str", "k2c", True), GATED]),
        "sel index outside its CSR row"),
    "src_id_out_of_range": (dict(files={"srcc": "srcbad"}, ops=[SPMV]), "src_id out of range"),
    "offsets_out_of_range": (dict(files={"offc": "offbad"}, ops=[SPMV]), "offsets out of range"),
    "offsets_zero_width": (dict(ops=[spmv(off="zz")]),
                           "offsets or src slot has width 0"),
    "x__dt__zero_width": (dict(ops=[spmv(x="zz")]),
                          "x slot (dt) has width 0"),
    "dst_and_offsets_both_unshaped": (
        dict(ops=[spmv("zz", "zo", nnz=False)]),
        "offsets or src slot has width 0"),
    "dst_too_small_for_n": (dict(shapes={"y": (2, 1)}, ops=[spmv(nnz=False)]),
                            "dst must be [n_neurons"),
    "nnz_needs_one_more_element": (dict(shapes={"y": (4, 1)}, ops=[SPMV]),
                                   "nnz needs dst to be"),
    "offsets_need_n_1_entries": (dict(shapes={"off": (1, 1)}, no_copy=("off",), ops=[SPMV]),
                                 "offsets must have n_neurons"),
    # examples/p16_compose/guards: the selgate set over the compose CSR
    "g_sel_odd_width": (dict(gate=True, data=COMPOSE, shapes={"sel": (4, 7)},
                             ops=[GATED]), "selgate needs an even sel width"),
    "g_sel_rows_short": (dict(gate=True, data=COMPOSE, shapes={"sel": (2, 8)},
                              ops=[GATED]), "sel table too small"),
    # (its .vml reads k from a slot it never shapes; here k comes from the
    # constant directly: k = 2 against one pair per row)
    "g_seg_k_too_big": (dict(gate=True, data=COMPOSE, shapes={"sel": (4, 2)},
                             ops=[("topk", "sel", "str", "k2c", True)]),
                        "k > dst segment width"),
}
# the negative controls: correct programs exit 0
OK_CASES = {
    "z_ok": (dict(ops=[SPMV], print=True), [1 * 10 + 2 * 20, 3 * 40, 0, 4 * 30, 4]),
    "g_ok": (dict(gate=True, data=COMPOSE, ops=[("topk", "sel", "str", "k2c", True),
                                                GATED], print=True),
             [1.49999988, 2.80000019, 3.50000000, 1.92499995, 8.0]),
}


def test_assembler_side_refusals():
    """The two cases the reference's assembler refuses (no image): a weight
    slot past 63 does not fit fl bits 0..5, and SPARSE_MATVEC needs its x
    operand. The program builder here encodes the weight slot in those bits,
    so a slot of 64 would alias the flags: the check that refuses it."""
    P = vmb.Program()
    for i in range(70):
        P.act(f"d{i:02d}", 1, 1)
    w = P.act("wz", 4, 1)
    assert w > vmb.SPARSE_WSLOT_MASK
    with pytest.raises(ValueError):
        vmb.sparse_matvec_fl(w, nnz=True)
    with pytest.raises(TypeError):
        vmb.sparse_matvec_fl()


@pytest.mark.parametrize("name", sorted(GUARDS))
def test_p16_guards_oracle(oracle, name):
    from test_vm_oracle import expect_exit
    case, msg = GUARDS[name]
    got = expect_exit(guard_program(case).build(), 9)
    assert msg in got, (name, got)


@pytest.mark.parametrize("name", sorted(OK_CASES))
def test_p16_ok_controls_oracle(oracle, name):
    case, want = OK_CASES[name]
    out, _ = oracle_run(guard_program(case))
    assert np.array_equal(bits(out), bits(np.float32(want)))


# ----------------------------------------------------------------- GPU
@pytest.fixture(scope="module")
def gvm(hip):
    import sparrow_amd
    from sparrow_amd import vm
    sparrow_amd.init(0)
    return vm


def gpu_run(gvm):
    def run(P, reads=()):
        with gvm.Vm(P.build()) as g:
            g.run()
            return g.output(), [g.read(r) for r in reads]
    return run


@pytest.mark.gpu
def test_p16_layer_gpu(gvm, oracle):
    check_layer(gpu_run(gvm))


@pytest.mark.gpu
def test_p16_guards_gpu(gvm, oracle):
    """Every guard program exits 9 on the GPU executor with the message the
    reference's probe expects, as the oracle does."""
    from sparrow_amd import VmlmError
    for name in sorted(GUARDS):
        case, msg = GUARDS[name]
        with pytest.raises(VmlmError) as e:
            with gvm.Vm(guard_program(case).build()) as g:
                g.run()
        assert e.value.code == 9 and msg in str(e.value), (name, str(e.value))
    for name, (case, want) in sorted(OK_CASES.items()):
        out, _ = gpu_run(gvm)(guard_program(case))
        assert np.array_equal(bits(out), bits(np.float32(want))), name

"""Writer and reader of .vmb program images, the binary the reference's
assembler emits (asm/src/main.rs:1196-1310) and its engine loads
(core/src/interp.rs:108-396, core/src/format.rs).

Layout (little-endian):
  header, 32 bytes: magic "VMLM" u32, version u16, pad u16, text_off, text_len,
      const_off, const_len, meta_off, meta_len (u32 each);
  TEXT: 16-byte instructions  op u8 | fl u8 | dt u16 | dst u32 | a u32 | b u32;
  CONST: every constant's bytes, each padded to 64 bytes;
  META: n_const, n_slot, slots_off, act_bytes, state_bytes, grad_bytes,
      names_off (u32 each; offsets relative to META), then the const table
      (24 bytes each: off, len, rows, cols u32, dtype u8, 3 pad, FNV-1a name
      hash u32), the slot table (16 bytes each: kind, idx, rows, cols u32)
      and one name hash per slot.

Activation, state and gradient slots are laid out in slot order, each at a
64-byte aligned offset of its region, as the assembler does. The opcode and
flag numbers are those of trans/src/opcode.rs.

`Program` builds images for tests and tools; the executor that runs them on
the GPU is `sparrow_amd.vm` (libvmlm_hip's vmlm_vm_*).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = 0x4D4C4D56
VERSION = 1
HEADER = 32
INS_SIZE = 16
CONST_ALIGN = 64
META_HDR = 28
CONST_ENT = 24
SLOT_ENT = 16

SLOT_CONST, SLOT_ACT, SLOT_STATE, SLOT_GRAD, SLOT_PARAM = 0, 1, 2, 3, 4
DT_F32, DT_F16, DT_I8, DT_I32, DT_BF16 = 0, 1, 2, 3, 4
DTYPES = {"f32": DT_F32, "f16": DT_F16, "i8": DT_I8, "i32": DT_I32, "bf16": DT_BF16}

# trans/src/opcode.rs
OP = dict(HALT=0, LOADK=1, COPY=2, RESHAPE=3, TRANSPOSE=4, CONCAT=5, SLICE=6, LAYERB=7,
          GEMM=10, BMM=11, OUTER=12, GEMV=13, EMB=14,
          EWADD=20, EWMUL=21, EWSUB=22, EWDIV=23, SCALE=24, ACT=25, EXP=26, LOG=27,
          CLAMP=28, NEG=29, LN=30, RMSNORM=31, SUM=32, MEAN=33, MAX=34, NORM=35,
          SOFTMAX=36, MASK_MUL=40, TOPK_THRESH=41, TOPK_IDX=42, GATHER=43, SCATTER=44,
          BRANCH=45, JMP=46, CMPLE=47, OP_CALL=48, SAVE=49, LOAD=50, PRINT=51, SHAPE=52,
          BIAS=53, GEMM_BWD_W=60, GEMM_BWD_X=61, BIAS_BWD=62, ACT_BWD=63, CE_BWD=64,
          MSE_BWD=65, ZERO=66, ADAM=67, SGD=68, LOSS_ADD=69, CLIP_GRAD=70, WRITECOL=71,
          EWMAX=72, GEMASK=73, SOFTMAX_BWD=80, LN_BWD=81, OUTER_BWD=82, EMB_BWD=83,
          ADAMW=84, LN_EPS=85, PUSH=86, POP=87, STACK_INIT=88, LOOP_CNT=89, ROPE=90,
          SIN=91, COS=92, TOPK_BY_STRENGTH=93, SPARSE_MATVEC=94)
FL_ACC, FL_TRANS_B, FL_BIAS, FL_BROADCAST, FL_CAUSAL, FL_NEG = 1, 2, 4, 8, 16, 32
FL_NNZ, FL_SELGATE = 1 << 6, 1 << 7
SPARSE_WSLOT_MASK = 0x3F
ACT = dict(relu=0, gelu=1, silu=2, sigmoid=3, tanh=4, relu2=5)

# Executor extensions (no reference counterpart; the reference unrolls
# decode because these operands are compile-time fields): the named slot
# holds the value as an f32 number instead.
FL_ROPE_POS_SLOT = 1 << 6      # ROPE: position from slot `fl`-less field `dt`... see vm docs
FL_WRITECOL_SLOT = 1 << 6      # WRITECOL: column offset from slot `dt`
FL_SOFTMAX_LIVE = 1 << 6       # SOFTMAX: live width from slot `b` (columns past it are 0)


def sparse_matvec_fl(wslot: int, nnz: bool = False, selgate: bool = False) -> int:
    """The `fl` byte of SPARSE_MATVEC: the weight slot in bits 0..5, FL_NNZ
    and FL_SELGATE above it. A weight slot past 63 does not fit, and the
    reference's assembler refuses such a program (no image is written)."""
    if not 0 <= wslot <= SPARSE_WSLOT_MASK:
        raise ValueError(f"SPARSE_MATVEC: weight slot {wslot} does not fit fl bits 0..5")
    return wslot | (FL_NNZ if nnz else 0) | (FL_SELGATE if selgate else 0)


def hash32(name: str) -> int:
    """FNV-1a 32-bit (core/src/format.rs hash32)."""
    h = 0x811C9DC5
    for c in name.encode():
        h ^= c
        h = (h * 0x01000193) & 0xFFFFFFFF
    return h


@dataclass
class Const:
    name: str
    data: bytes
    rows: int
    cols: int
    dtype: int


@dataclass
class Slot:
    name: str
    kind: int
    rows: int
    cols: int


@dataclass
class Program:
    consts: list = field(default_factory=list)
    slots: list = field(default_factory=list)
    text: list = field(default_factory=list)
    index: dict = field(default_factory=dict)

    # -------------------------------------------------------------- slots
    def _slot(self, name, kind, rows, cols):
        if name in self.index:
            s = self.slots[self.index[name]]
            if (s.kind, s.rows, s.cols) != (kind, rows, cols):
                raise ValueError(f"slot {name} redeclared")
            return self.index[name]
        self.index[name] = len(self.slots)
        self.slots.append(Slot(name, kind, int(rows), int(cols)))
        return self.index[name]

    def const(self, name, array, dtype="f32", rows=None, cols=None, kind=SLOT_CONST):
        """A constant slot; `array` is raw values of `dtype` (bf16 as uint16
        bits, i8 as int8). rows x cols default to the array's 2-D shape."""
        dt = DTYPES[dtype] if isinstance(dtype, str) else int(dtype)
        a = np.ascontiguousarray(array)
        if rows is None:
            shp = a.shape if a.ndim == 2 else (1, a.size)
            rows, cols = shp
        self.consts.append(Const(name, a.tobytes(), int(rows), int(cols), dt))
        return self._slot(name, kind, rows, cols)

    def scalar(self, name, value):
        return self.const(name, np.float32([value]), "f32", 1, 1)

    def act(self, name, rows, cols):
        return self._slot(name, SLOT_ACT, rows, cols)

    def state(self, name, rows, cols):
        return self._slot(name, SLOT_STATE, rows, cols)

    def grad(self, name, rows, cols):
        return self._slot(name, SLOT_GRAD, rows, cols)

    def __getitem__(self, name):
        return self.index[name]

    # -------------------------------------------------------------- text
    def ins(self, op, dst=0, a=0, b=0, dt=0, fl=0):
        op = OP[op] if isinstance(op, str) else int(op)
        self.text.append((op, int(fl) & 0xFF, int(dt) & 0xFFFF, int(dst), int(a), int(b)))
        return len(self.text) - 1

    def label(self):
        """Index of the next instruction (a jump target)."""
        return len(self.text)

    # -------------------------------------------------------------- image
    def build(self) -> bytes:
        # constant offsets (each constant starts on a CONST_ALIGN boundary);
        # the pool itself is written once into the final image below
        offs, clen = [], 0
        for c in self.consts:
            offs.append(clen)
            clen += (len(c.data) + CONST_ALIGN - 1) // CONST_ALIGN * CONST_ALIGN
        cidx = {c.name: i for i, c in enumerate(self.consts)}
        region = {SLOT_ACT: 0, SLOT_STATE: 0, SLOT_GRAD: 0}
        idx = []
        for s in self.slots:
            if s.kind in (SLOT_CONST, SLOT_PARAM):
                idx.append(cidx[s.name])
            else:
                idx.append(region[s.kind])
                region[s.kind] = (region[s.kind] + s.rows * s.cols * 4 + 63) & ~63
        slots_off = META_HDR + len(self.consts) * CONST_ENT
        names_off = slots_off + len(self.slots) * SLOT_ENT
        meta = bytearray(struct.pack("<7I", len(self.consts), len(self.slots), slots_off,
                                     region[SLOT_ACT], region[SLOT_STATE], region[SLOT_GRAD],
                                     names_off))
        for c, off in zip(self.consts, offs):
            meta += struct.pack("<4IB3xI", off, len(c.data), c.rows, c.cols, c.dtype,
                                hash32(c.name))
        for s, i in zip(self.slots, idx):
            meta += struct.pack("<4I", s.kind, i, s.rows, s.cols)
        for s in self.slots:
            meta += struct.pack("<I", hash32(s.name))
        ins = struct.Struct("<BBHIII")
        text = bytearray(ins.size * len(self.text))
        for i, t in enumerate(self.text):
            ins.pack_into(text, i * ins.size, *t)
        text_off = HEADER
        const_off = text_off + len(text)
        meta_off = const_off + clen
        head = struct.pack("<IHHIIIIII", MAGIC, VERSION, 0, text_off, len(text), const_off,
                           clen, meta_off, len(meta))
        # one join: the image is allocated and written once
        parts = [head, bytes(text)]
        for c in self.consts:
            parts.append(c.data)
            pad = -len(c.data) % CONST_ALIGN
            if pad:
                parts.append(bytes(pad))
        parts.append(bytes(meta))
        return b"".join(parts)


def parse(image: bytes) -> dict:
    """Header, instructions, const table and slot table of an image (for
    inspection and tests)."""
    magic, ver, _, text_off, text_len, const_off, const_len, meta_off, meta_len = \
        struct.unpack_from("<IHHIIIIII", image, 0)
    text = [struct.unpack_from("<BBHIII", image, text_off + i * INS_SIZE)
            for i in range(text_len // INS_SIZE)]
    n_const, n_slot, slots_off, act_b, state_b, grad_b, names_off = \
        struct.unpack_from("<7I", image, meta_off)
    consts = [struct.unpack_from("<4IB3xI", image, meta_off + META_HDR + i * CONST_ENT)
              for i in range(n_const)]
    slots = [struct.unpack_from("<4I", image, meta_off + slots_off + i * SLOT_ENT)
             for i in range(n_slot)]
    names = [struct.unpack_from("<I", image, meta_off + names_off + 4 * i)[0]
             for i in range(n_slot)]
    return dict(magic=magic, version=ver, text=text, const_off=const_off, const_len=const_len,
                consts=consts, slots=slots, names=names, act_bytes=act_b, state_bytes=state_b,
                grad_bytes=grad_b)

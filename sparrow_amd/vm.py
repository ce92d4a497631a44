"""The device-resident VM executor (libvmlm_hip vmlm_vm_*): load a .vmb
image (core/src/interp.rs Vm::load / load_weights_mapped), run it on the GPU
(Vm::run), and move f32 slot values and PRINT output to the host.

Failures raise sparrow_amd.VmlmError carrying the interpreter's exit code.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import check, lib


class Vm:
    def __init__(self, image: bytes, weights: np.ndarray | None = None):
        self._h = None
        self._image = bytes(image)
        self._weights = weights  # the mapped region must stay alive
        h = C.c_void_p()
        wp = weights.ctypes.data if weights is not None else None
        wl = weights.nbytes if weights is not None else 0
        check(lib().vmlm_vm_load(self._image, len(self._image), wp, wl, C.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().vmlm_vm_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run(self):
        check(lib().vmlm_vm_run(self._h))

    def slot_index(self, name: str) -> int:
        i = C.c_uint32()
        check(lib().vmlm_vm_find_slot(self._h, name.encode(), C.byref(i)))
        return i.value

    def shape(self, slot) -> tuple:
        i = slot if isinstance(slot, int) else self.slot_index(slot)
        r, c, dt = C.c_uint32(), C.c_uint32(), C.c_uint8()
        check(lib().vmlm_vm_slot_info(self._h, i, None, C.byref(r), C.byref(c), C.byref(dt)))
        return r.value, c.value

    def read(self, slot) -> np.ndarray:
        i = slot if isinstance(slot, int) else self.slot_index(slot)
        r, c = self.shape(i)
        out = np.empty((r, c), np.float32)
        check(lib().vmlm_vm_read_slot(self._h, i, out.ctypes.data, out.size))
        return out

    def write(self, slot, values) -> None:
        i = slot if isinstance(slot, int) else self.slot_index(slot)
        v = np.ascontiguousarray(values, np.float32).ravel()
        check(lib().vmlm_vm_write_slot(self._h, i, v.ctypes.data, v.size))

    def output(self) -> np.ndarray:
        n = C.c_size_t()
        check(lib().vmlm_vm_output(self._h, None, 0, C.byref(n)))
        out = np.empty(n.value, np.float32)
        check(lib().vmlm_vm_output(self._h, out.ctypes.data, out.size, C.byref(n)))
        return out

    def clear_output(self) -> None:
        check(lib().vmlm_vm_clear_output(self._h))

    def fused_runs(self) -> int:
        """Opcode runs executed as one launch each (found at load)."""
        n = C.c_size_t()
        check(lib().vmlm_vm_fused_runs(self._h, C.byref(n)))
        return n.value

    def fused_opcodes(self) -> int:
        """Opcodes those runs cover."""
        n = C.c_size_t()
        check(lib().vmlm_vm_fused_opcodes(self._h, C.byref(n)))
        return n.value

    def set_graphs(self, on: bool) -> None:
        """Replay loop bodies as HIP graphs (the default), or run every
        opcode one by one; the results are the same bits."""
        check(lib().vmlm_vm_set_graphs(self._h, 1 if on else 0))

    def graph_segments(self) -> int:
        """Loop bodies replayed as HIP graphs so far."""
        n = C.c_size_t()
        check(lib().vmlm_vm_graph_segments(self._h, C.byref(n)))
        return n.value

    def swizzled_consts(self) -> int:
        """int8 constants also held in the swizzled MFMA layout, which
        OP_GEMM reads instead of the row-major bytes."""
        n = C.c_size_t()
        check(lib().vmlm_vm_swizzled_consts(self._h, C.byref(n)))
        return n.value


def pool_uploads() -> int:
    n = C.c_size_t()
    check(lib().vmlm_vm_pool_uploads(C.byref(n)))
    return n.value

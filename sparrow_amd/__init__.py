"""sparrow_amd -- MI355X (gfx950) backend for VMLM's inference hot path.

The product is the C-ABI library libvmlm_hip.so (include/vmlm_hip.h); this
package loads it with ctypes and mirrors the vmlm-ops kernel interface
(sparrow_amd.ops), the B1 connection type (sparrow_amd.conn) and the
MiniCPM-shaped decoder session (sparrow_amd.decoder).

There is no CPU fallback: every entry point calls the HIP library, and
loading fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libvmlm_hip.so"

_lib = None


class VmlmError(RuntimeError):
    """A non-zero status from libvmlm_hip (2 device, 5 unimplemented,
    9 guard violation -- the reference engine's exit codes)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"vmlm status {code}: {msg}")
        self.code = code


def lib() -> C.CDLL:
    """Load libvmlm_hip.so (built by `python -m sparrow_amd.build`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m sparrow_amd.build` "
                          "(there is no CPU fallback)")
    L = C.CDLL(str(LIB_PATH))
    from . import _abi
    _abi.declare(L)
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().vmlm_hip_last_error().decode(errors="replace")
        raise VmlmError(rc, msg)


def init(device: int = 0) -> None:
    check(lib().vmlm_hip_init(device))


def sync() -> None:
    check(lib().vmlm_hip_sync())

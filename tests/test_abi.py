"""CPU checks of the C-ABI boundary: libvmlm_hip.so loads without a GPU and
exports every function include/vmlm_hip.h declares; the ctypes table covers
the same set. No compute calls (there is no GPU here)."""
import ctypes as C
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "vmlm_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(vmlm_\w+)\s*\(", text))
    # function-pointer fields inside the backend struct are not exports
    return {n for n in names if not n.endswith("_t")}


def test_library_exports_every_declared_symbol():
    import sparrow_amd
    L = C.CDLL(str(sparrow_amd.LIB_PATH))
    missing = [n for n in sorted(header_functions()) if not hasattr(L, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_ctypes_table_matches_header():
    from sparrow_amd import _abi
    declared = header_functions()
    assert set(_abi.SIGNATURES) == declared


def test_loader_declares_all():
    import sparrow_amd
    L = sparrow_amd.lib()
    assert L.vmlm_hip_version().decode().startswith("vmlm_hip")


def test_status_codes_match_reference_exit_codes():
    """runtime/src/main.rs:15-19: 2 I/O, 5 unimplemented op, 9 guard."""
    text = (ROOT / "include" / "vmlm_hip.h").read_text()
    assert "#define VMLM_ERR_DEVICE 2" in text
    assert "#define VMLM_ERR_UNIMPL 5" in text
    assert "#define VMLM_ERR_GUARD 9" in text


def test_no_oracle_in_product_path():
    """The product package never imports or loads the oracle."""
    for p in (ROOT / "sparrow_amd").rglob("*.py"):
        src = p.read_text()
        assert "oracle" not in src.replace("oracle/", ""), p
    for p in (ROOT / "sparrow_amd" / "csrc").glob("*"):
        assert "vmlm_oracle" not in p.read_text(), p


def _header_params():
    """name -> parameter count of every function include/vmlm_hip.h declares."""
    text = (ROOT / "include" / "vmlm_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(vmlm_\w+)\s*\(([^;{]*?)\)\s*;", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_ffi_crate_matches_header():
    """ffi/vmlm-ops-hip/src/lib.rs (the Rust FFI crate; no Rust toolchain
    here, so it is checked as text): every C function its extern block
    declares exists in include/vmlm_hip.h with the same parameter count, and
    the library exports it."""
    import sparrow_amd
    src = (ROOT / "ffi" / "vmlm-ops-hip" / "src" / "lib.rs").read_text()
    block = src[src.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    decls = re.findall(r"fn\s+(vmlm_\w+)\s*\(([^)]*)\)", block, flags=re.S)
    assert len(decls) >= 30
    # the device VM's entry points, which the runtime's load -> run path binds
    # (runtime/src/main.rs:136-153, 209-260)
    vm_needed = {"vmlm_vm_load", "vmlm_vm_destroy", "vmlm_vm_run", "vmlm_vm_find_slot",
                 "vmlm_vm_slot_info", "vmlm_vm_write_slot", "vmlm_vm_read_slot",
                 "vmlm_vm_output", "vmlm_vm_clear_output"}
    assert vm_needed <= {name for name, _ in decls}, vm_needed - {name for name, _ in decls}
    for fn in ("pub unsafe fn load(", "pub unsafe fn run(", "pub unsafe fn slot_index(",
               "pub unsafe fn write_slot(", "impl Drop for DeviceVm"):
        assert fn in src, fn
    header = _header_params()
    L = C.CDLL(str(sparrow_amd.LIB_PATH))
    for name, args in decls:
        n = 0 if not args.strip() else args.count(":")
        assert name in header, name
        assert header[name] == n, (name, header[name], n)
        assert hasattr(L, name), name

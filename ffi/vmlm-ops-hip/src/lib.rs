//! `vmlm-ops-hip`: the MI355X (gfx950) kernels of libvmlm_hip.so under the
//! names and signatures of `vmlm_ops::kernels` (ops/src/kernels.rs), so that
//! the interpreter, the JIT glue and the model code call them unchanged.
//!
//! The C declarations below mirror include/vmlm_hip.h one for one. Every C
//! call returns a status; `check` turns a non-zero one into the
//! interpreter's print-and-exit (core/src/interp.rs:2357-2376): 9 guard,
//! 5 unsupported, 2 device or runtime failure.
//!
//! Swap inside vmlm-ops (ops/src/lib.rs), with a `hip` feature that depends
//! on this crate. Names imported explicitly shadow the glob, so only the
//! hot-path kernels move to the GPU and every other item stays the CPU code:
//!
//! ```ignore
//! #[cfg(not(feature = "hip"))]
//! pub mod kernels;
//! #[cfg(feature = "hip")]
//! #[path = "kernels.rs"]
//! mod kernels_cpu;
//! #[cfg(feature = "hip")]
//! pub mod kernels {
//!     pub use super::kernels_cpu::*;
//!     pub use vmlm_ops_hip::{act_avx2, ew_op, gemm, gemm_nt, gemm_nt_bf16, gemm_nt_int8,
//!                            jit_act, jit_bias, jit_ewadd, jit_ewdiv, jit_ewmul, jit_ewsub,
//!                            jit_gemm_nt, jit_ln, jit_outer, jit_softmax, layernorm, outer,
//!                            rmsnorm, softmax, transpose_t8_avx2, transpose_t8_back_avx2};
//! }
//! ```
//!
//! The CPU file keeps its `#[no_mangle]` jit_* symbols; the JIT takes the
//! addresses of the `kernels::jit_*` paths (trans/src/jit.rs:185, 252), which
//! now resolve to the functions here. `b1_pure::b1_forward` / `b1_forward_t8`
//! (ops/src/b1_pure.rs:151, 271) take `&SparseConnW`; under the feature they
//! forward to `b1_forward_c` / `b1_forward_t8_c` with `SparseConnWC::from`
//! the struct's fields (shown at the end of this file).
#![no_std]
#![allow(clippy::missing_safety_doc, clippy::too_many_arguments)]

use core::ffi::{c_char, c_int, c_void};

/// vmlm_sparse_conn_w: the fields of ops/src/conn.rs:8-53 `SparseConnW` in
/// order, laid out for C.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct SparseConnWC {
    pub e: usize,
    pub k0: usize,
    pub layer: u32,
    pub n_neurons: u32,
    pub w: *mut f32,
    pub src: *mut f32,
    pub src_u32: *mut u32,
    pub act: *mut f32,
}

/// The library's device-resident VM (`vmlm_vm` in include/vmlm_hip.h); only
/// ever handled by pointer.
#[repr(C)]
pub struct VmRaw {
    _opaque: [u8; 0],
}

/// vmlm_backend_t: sys/src/lib.rs:29-38 `Backend`, field for field.
pub type HipBackend = vmlm_sys::Backend;

extern "C" {
    fn vmlm_hip_last_error() -> *const c_char;
    fn vmlm_gemm_nt_int8(a: *const f32, q: *const i8, scale: *const f32, c: *mut f32,
                         m: usize, n: usize, k: usize) -> c_int;
    fn vmlm_gemm_nt_bf16(a: *const f32, b: *const u16, c: *mut f32, m: usize, n: usize,
                         k: usize) -> c_int;
    fn vmlm_gemm_nt(a: *const f32, b: *const f32, c: *mut f32, m: usize, n: usize, k: usize,
                    acc: bool) -> c_int;
    fn vmlm_gemm(a: *const f32, b: *const f32, c: *mut f32, m: usize, n: usize, k: usize,
                 acc: bool) -> c_int;
    fn vmlm_rmsnorm(dst: *mut f32, src: *const f32, g: *const f32, rows: usize, cols: usize,
                    eps: f32) -> c_int;
    fn vmlm_softmax(p: *mut f32, rows: usize, cols: usize, causal: bool) -> c_int;
    fn vmlm_act(dst: *mut f32, n: usize, kind: u16) -> c_int;
    fn vmlm_ew_op(dst: *mut f32, x: *const f32, y: *const f32, n: usize, op: u8) -> c_int;
    fn vmlm_layernorm(x: *mut f32, g: *const f32, b: *const f32, rows: usize, cols: usize,
                      eps: f32) -> c_int;
    fn vmlm_outer(s: *mut f32, v: *const f32, k: *const f32, m: usize, n: usize,
                  sc: f32) -> c_int;
    fn vmlm_b1_forward(sc: *const SparseConnWC, x: *const f32, y: *mut f32,
                       macs: *mut usize) -> c_int;
    fn vmlm_b1_forward_t8(sc: *const SparseConnWC, xt: *const f32, t8: usize, n_tokens: usize,
                          yt: *mut f32, macs: *mut usize) -> c_int;
    fn vmlm_transpose_t8(x: *const f32, t: usize, d: usize, xt: *mut f32, t8: usize) -> c_int;
    fn vmlm_transpose_t8_back(a: *const f32, rows: usize, cols: usize, out: *mut f32,
                              os: usize, in_stride: usize) -> c_int;
    fn vmlm_jit_gemm_nt(a: *const f32, b: *const f32, c: *mut f32, dims: u64) -> c_int;
    fn vmlm_jit_act(p: *mut f32, n: usize, kind: u64) -> c_int;
    fn vmlm_jit_ewadd(d: *mut f32, x: *const f32, y: *const f32, n: usize) -> c_int;
    fn vmlm_jit_ewmul(d: *mut f32, x: *const f32, y: *const f32, n: usize) -> c_int;
    fn vmlm_jit_ewsub(d: *mut f32, x: *const f32, y: *const f32, n: usize) -> c_int;
    fn vmlm_jit_ewdiv(d: *mut f32, x: *const f32, y: *const f32, n: usize) -> c_int;
    fn vmlm_jit_bias(d: *mut f32, b: *const f32, rows: usize, cols: usize) -> c_int;
    fn vmlm_jit_ln(x: *mut f32, g: *const f32, b: *const f32, dims: u64, pad: u64) -> c_int;
    fn vmlm_jit_softmax(p: *mut f32, dims: u64, causal: u64) -> c_int;
    fn vmlm_jit_outer(s: *mut f32, v: *const f32, k: *const f32, dims: u64) -> c_int;
    fn vmlm_backend_dot256(a: *const f32, b: *const f32, n: usize) -> f32;
    fn vmlm_backend_axpy256(y: *mut f32, x: *const f32, a: f32, n: usize);
    fn vmlm_backend_add256(y: *mut f32, x: *const f32, n: usize);
    fn vmlm_backend_max256(x: *const f32, n: usize) -> f32;
    fn vmlm_backend_sum256(x: *const f32, n: usize) -> f32;
    fn vmlm_backend_scale_mul(dst: *mut f32, src: *const f32, a: f32, n: usize);
    fn vmlm_vm_load(image: *const u8, len: usize, weights: *const u8, weights_len: usize,
                    out: *mut *mut VmRaw) -> c_int;
    fn vmlm_vm_destroy(vm: *mut VmRaw) -> c_int;
    fn vmlm_vm_run(vm: *mut VmRaw) -> c_int;
    fn vmlm_vm_find_slot(vm: *const VmRaw, name: *const c_char, slot: *mut u32) -> c_int;
    fn vmlm_vm_slot_info(vm: *mut VmRaw, slot: u32, dptr: *mut *mut c_void, rows: *mut u32,
                         cols: *mut u32, dtype: *mut u8) -> c_int;
    fn vmlm_vm_write_slot(vm: *mut VmRaw, slot: u32, host: *const f32, count: usize) -> c_int;
    fn vmlm_vm_read_slot(vm: *mut VmRaw, slot: u32, host: *mut f32, count: usize) -> c_int;
    fn vmlm_vm_output(vm: *mut VmRaw, host: *mut f32, cap: usize, count: *mut usize) -> c_int;
    fn vmlm_vm_clear_output(vm: *mut VmRaw) -> c_int;
}

/// The interpreter's error convention: print the library's message and exit
/// with the status.
#[inline]
fn check(rc: c_int) {
    if rc != 0 {
        unsafe {
            let msg = vmlm_hip_last_error();
            let mut n = 0usize;
            while *msg.add(n) != 0 {
                n += 1;
            }
            vmlm_sys::io::print(core::slice::from_raw_parts(msg as *const u8, n));
            vmlm_sys::io::print(b"\n");
            vmlm_sys::io::exit(rc)
        }
    }
}

// ---------------------------------------------------------------- kernels
/// ops/src/kernels.rs:1258
pub unsafe fn gemm_nt_int8(a: *const f32, q: *const i8, scale: *const f32, c: *mut f32,
                           m: usize, n: usize, k: usize) {
    check(vmlm_gemm_nt_int8(a, q, scale, c, m, n, k))
}
/// ops/src/kernels.rs:1202
pub unsafe fn gemm_nt_bf16(a: *const f32, b: *const u16, c: *mut f32, m: usize, n: usize,
                           k: usize) {
    check(vmlm_gemm_nt_bf16(a, b, c, m, n, k))
}
/// ops/src/kernels.rs:987
pub unsafe fn gemm_nt(a: *const f32, b: *const f32, c: *mut f32, m: usize, n: usize, k: usize,
                      acc: bool) {
    check(vmlm_gemm_nt(a, b, c, m, n, k, acc))
}
/// ops/src/kernels.rs:407
pub unsafe fn gemm(a: *const f32, b: *const f32, c: *mut f32, m: usize, n: usize, k: usize,
                   acc: bool) {
    check(vmlm_gemm(a, b, c, m, n, k, acc))
}
/// ops/src/kernels.rs:1346
pub unsafe fn rmsnorm(dst: *mut f32, src: *const f32, g: *const f32, rows: usize, cols: usize,
                      eps: f32) {
    check(vmlm_rmsnorm(dst, src, g, rows, cols, eps))
}
/// ops/src/kernels.rs:1389
pub unsafe fn softmax(p: *mut f32, rows: usize, cols: usize, causal: bool) {
    check(vmlm_softmax(p, rows, cols, causal))
}
/// ops/src/kernels.rs:1146
pub unsafe fn act_avx2(dst: *mut f32, n: usize, kind: u16) {
    check(vmlm_act(dst, n, kind))
}
/// ops/src/kernels.rs:1117
pub unsafe fn ew_op(dst: *mut f32, x: *const f32, y: *const f32, n: usize, op: u8) {
    check(vmlm_ew_op(dst, x, y, n, op))
}
/// ops/src/kernels.rs:1308
pub unsafe fn layernorm(x: *mut f32, g: *const f32, b: *const f32, rows: usize, cols: usize,
                        eps: f32) {
    check(vmlm_layernorm(x, g, b, rows, cols, eps))
}
/// ops/src/kernels.rs:1436
pub unsafe fn outer(s: *mut f32, v: *const f32, k: *const f32, m: usize, n: usize, sc: f32) {
    check(vmlm_outer(s, v, k, m, n, sc))
}
/// ops/src/kernels.rs:1881
pub unsafe fn transpose_t8_avx2(x: *const f32, t: usize, d: usize, xt: *mut f32, t8: usize) {
    check(vmlm_transpose_t8(x, t, d, xt, t8))
}
/// ops/src/kernels.rs:3307
pub unsafe fn transpose_t8_back_avx2(a: *const f32, rows: usize, cols: usize, out: *mut f32,
                                     os: usize, in_stride: usize) {
    check(vmlm_transpose_t8_back(a, rows, cols, out, os, in_stride))
}

/// ops/src/b1_pure.rs:151 on the C layout of `SparseConnW`; returns the MACs.
pub unsafe fn b1_forward_c(sc: &SparseConnWC, x: *const f32, y: *mut f32) -> usize {
    let mut macs = 0usize;
    check(vmlm_b1_forward(sc, x, y, &mut macs));
    macs
}
/// ops/src/b1_pure.rs:271 on the C layout of `SparseConnW`; returns the MACs.
pub unsafe fn b1_forward_t8_c(sc: &SparseConnWC, xt: *const f32, t8: usize, n_tokens: usize,
                              yt: *mut f32) -> usize {
    let mut macs = 0usize;
    check(vmlm_b1_forward_t8(sc, xt, t8, n_tokens, yt, &mut macs));
    macs
}

// ---------------------------------------------------------------- JIT glue
// ops/src/kernels.rs:1017-1093, same extern "system" signatures (without
// #[no_mangle]: the JIT takes these addresses through the kernels paths).
pub unsafe extern "system" fn jit_gemm_nt(a: *const f32, b: *const f32, c: *mut f32, dims: u64) {
    check(vmlm_jit_gemm_nt(a, b, c, dims))
}
pub unsafe extern "system" fn jit_act(p: *mut f32, n: usize, kind: u64) {
    check(vmlm_jit_act(p, n, kind))
}
pub unsafe extern "system" fn jit_ewadd(d: *mut f32, x: *const f32, y: *const f32, n: usize) {
    check(vmlm_jit_ewadd(d, x, y, n))
}
pub unsafe extern "system" fn jit_ewmul(d: *mut f32, x: *const f32, y: *const f32, n: usize) {
    check(vmlm_jit_ewmul(d, x, y, n))
}
pub unsafe extern "system" fn jit_ewsub(d: *mut f32, x: *const f32, y: *const f32, n: usize) {
    check(vmlm_jit_ewsub(d, x, y, n))
}
pub unsafe extern "system" fn jit_ewdiv(d: *mut f32, x: *const f32, y: *const f32, n: usize) {
    check(vmlm_jit_ewdiv(d, x, y, n))
}
pub unsafe extern "system" fn jit_bias(d: *mut f32, b: *const f32, rows: usize, cols: usize) {
    check(vmlm_jit_bias(d, b, rows, cols))
}
pub unsafe extern "system" fn jit_ln(x: *mut f32, g: *const f32, b: *const f32, dims: u64,
                                     pad: u64) {
    check(vmlm_jit_ln(x, g, b, dims, pad))
}
pub unsafe extern "system" fn jit_softmax(p: *mut f32, dims: u64, causal: u64) {
    check(vmlm_jit_softmax(p, dims, causal))
}
pub unsafe extern "system" fn jit_outer(s: *mut f32, v: *const f32, k: *const f32, dims: u64) {
    check(vmlm_jit_outer(s, v, k, dims))
}

// ---------------------------------------------------------------- Backend
/// The GPU `Backend` table (sys/src/lib.rs:29-38): the library's functions
/// take device pointers in place and stage host pointers.
pub fn hip_backend() -> HipBackend {
    vmlm_sys::Backend {
        name: b"hip_gfx950\0".as_ptr(),
        dot256: vmlm_backend_dot256,
        axpy256: vmlm_backend_axpy256,
        add256: vmlm_backend_add256,
        max256: vmlm_backend_max256,
        sum256: vmlm_backend_sum256,
        scale_mul: vmlm_backend_scale_mul,
    }
}

// The adapter for ops/src/b1_pure.rs under the `hip` feature (SparseConnW is
// Copy and its fields are public):
//
//     #[cfg(feature = "hip")]
//     pub unsafe fn b1_forward(sc: &SparseConnW, x: *const f32, y: *mut f32) -> usize {
//         vmlm_ops_hip::b1_forward_c(&c_layout(sc), x, y)
//     }
//     fn c_layout(sc: &SparseConnW) -> vmlm_ops_hip::SparseConnWC {
//         vmlm_ops_hip::SparseConnWC { e: sc.e, k0: sc.k0, layer: sc.layer,
//             n_neurons: sc.n_neurons, w: sc.w, src: sc.src, src_u32: sc.src_u32, act: sc.act }
//     }

// ---------------------------------------------------------------- device VM
/// A `.vmb` program loaded onto the GPU: the counterpart of `Vm::load` +
/// `Vm::run` (core/src/interp.rs:108-396, 720-2370). The constant pool is
/// uploaded once (shared by every VM loaded over the same weights), the
/// activation / state / gradient arenas live in HBM, and every opcode runs
/// as GPU kernels on the VM's stream with the interpreter's guards. Failures
/// take the interpreter's exit path through `check` with its exit codes
/// (9 guard, 5 unimplemented op, 6 training op, 3 bad magic, 7 slot not
/// found, 8 EW shape mismatch, 2 device).
pub struct DeviceVm {
    raw: *mut VmRaw,
}

impl DeviceVm {
    /// `Vm::load(buf)` (core/src/interp.rs:108): parses the image, runs
    /// `audit_const_dtypes` and `bind_slots`, uploads the CONST region.
    pub unsafe fn load(image: *const u8, len: usize) -> DeviceVm {
        let mut raw = core::ptr::null_mut();
        check(vmlm_vm_load(image, len, core::ptr::null(), 0, &mut raw));
        DeviceVm { raw }
    }
    /// `load_weights_mapped` (core/src/interp.rs:108-236): the constants come
    /// from a separately mapped weights region, uploaded once per (pointer,
    /// length) and shared; the caller keeps it unchanged while VMs use it.
    pub unsafe fn load_mapped(image: *const u8, len: usize, weights: *const u8,
                              weights_len: usize) -> DeviceVm {
        let mut raw = core::ptr::null_mut();
        check(vmlm_vm_load(image, len, weights, weights_len, &mut raw));
        DeviceVm { raw }
    }
    /// `Vm::run` (core/src/interp.rs:720): runs to HALT, then prints every
    /// value the program's PRINT instructions produced, in order, in the
    /// interpreter's format (`print_f32`), before a failing status exits.
    pub unsafe fn run(&mut self) {
        let rc = vmlm_vm_run(self.raw);
        self.flush_prints();
        check(rc);
    }
    unsafe fn flush_prints(&mut self) {
        let mut n = 0usize;
        check(vmlm_vm_output(self.raw, core::ptr::null_mut(), 0, &mut n));
        if n == 0 {
            return;
        }
        let buf = vmlm_sys::mem::alloc(n * 4) as *mut f32;
        let mut got = 0usize;
        check(vmlm_vm_output(self.raw, buf, n, &mut got));
        vmlm_sys::io::print_f32(buf, if got < n { got } else { n });
        vmlm_sys::mem::dealloc(buf as *mut u8, n * 4);
        check(vmlm_vm_clear_output(self.raw));
    }
    /// The slot named `name` (NUL-terminated), or None when the program
    /// declares no such slot: the runtime's `slot_index` probe
    /// (runtime/src/main.rs:160-190), which must not exit on a miss.
    pub unsafe fn slot_index(&self, name: &[u8]) -> Option<u32> {
        let mut slot = 0u32;
        match vmlm_vm_find_slot(self.raw, name.as_ptr() as *const c_char, &mut slot) {
            0 => Some(slot),
            7 => None,
            rc => {
                check(rc);
                None
            }
        }
    }
    /// `Vm::slot_shape` (rows, cols).
    pub unsafe fn slot_shape(&self, slot: u32) -> (usize, usize) {
        let (mut r, mut c) = (0u32, 0u32);
        check(vmlm_vm_slot_info(self.raw, slot, core::ptr::null_mut(), &mut r, &mut c,
                                core::ptr::null_mut()));
        (r as usize, c as usize)
    }
    /// Device address of a slot (layer base applied), for callers that run
    /// their own kernels on the VM's arenas.
    pub unsafe fn slot_device_ptr(&self, slot: u32) -> *mut c_void {
        let mut p = core::ptr::null_mut();
        check(vmlm_vm_slot_info(self.raw, slot, &mut p, core::ptr::null_mut(),
                                core::ptr::null_mut(), core::ptr::null_mut()));
        p
    }
    /// Host f32 values into an activation / state / gradient slot: what
    /// `load_ids` does through `slot_mut` (runtime/src/main.rs:209-247).
    pub unsafe fn write_slot(&mut self, slot: u32, host: *const f32, count: usize) {
        check(vmlm_vm_write_slot(self.raw, slot, host, count))
    }
    /// A slot's first `count` f32 values back to the host.
    pub unsafe fn read_slot(&self, slot: u32, host: *mut f32, count: usize) {
        check(vmlm_vm_read_slot(self.raw, slot, host, count))
    }
}

impl Drop for DeviceVm {
    fn drop(&mut self) {
        unsafe {
            vmlm_vm_destroy(self.raw);
        }
    }
}

"""ctypes declarations of include/vmlm_hip.h (kept in the header's order)."""
from __future__ import annotations

import ctypes as C

P = C.c_void_p
SZ = C.c_size_t
I = C.c_int
F = C.c_float
B = C.c_bool
U16 = C.c_uint16
U8 = C.c_uint8
U32 = C.c_uint32
U64 = C.c_uint64


class SparseConnW(C.Structure):
    """ops/src/conn.rs:8-53 SparseConnW, as vmlm_sparse_conn_w."""
    _fields_ = [("e", SZ), ("k0", SZ), ("layer", U32), ("n_neurons", U32),
                ("w", P), ("src", P), ("src_u32", P), ("act", P)]


class Backend(C.Structure):
    """sys/src/lib.rs:29-38 Backend, as vmlm_backend_t."""
    _fields_ = [("name", C.c_char_p),
                ("dot256", C.CFUNCTYPE(F, P, P, SZ)),
                ("axpy256", C.CFUNCTYPE(None, P, P, F, SZ)),
                ("add256", C.CFUNCTYPE(None, P, P, SZ)),
                ("max256", C.CFUNCTYPE(F, P, SZ)),
                ("sum256", C.CFUNCTYPE(F, P, SZ)),
                ("scale_mul", C.CFUNCTYPE(None, P, P, F, SZ))]


class DecoderCfg(C.Structure):
    _fields_ = [("n_layers", U32), ("hidden", U32), ("n_heads", U32), ("head_dim", U32),
                ("inter", U32), ("vocab", U32), ("batch", U32), ("cap", U32),
                ("eps", F), ("theta", F), ("attn_scale", F)]


SIGNATURES = {
    # library
    "vmlm_hip_init": (I, [I]),
    "vmlm_hip_last_error": (C.c_char_p, []),
    "vmlm_hip_version": (C.c_char_p, []),
    "vmlm_hip_sync": (I, []),
    "vmlm_hip_malloc": (I, [C.POINTER(P), SZ]),
    "vmlm_hip_free": (I, [P]),
    "vmlm_hip_memcpy_h2d": (I, [P, P, SZ]),
    "vmlm_hip_memcpy_d2h": (I, [P, P, SZ]),
    "vmlm_hip_memcpy_d2d": (I, [P, P, SZ]),
    "vmlm_hip_memset": (I, [P, I, SZ]),
    "vmlm_hip_event_record": (I, [P, C.POINTER(I)]),
    "vmlm_hip_event_elapsed_ms": (I, [I, I, C.POINTER(F)]),
    "vmlm_hip_event_release_all": (I, []),
    "vmlm_hip_capture_begin": (I, [P]),
    "vmlm_hip_capture_end": (I, [P, C.POINTER(P)]),
    "vmlm_hip_graph_launch": (I, [P, P]),
    "vmlm_hip_graph_destroy": (I, [P]),
    # layer 1
    "vmlm_gemm_nt_int8": (I, [P, P, P, P, SZ, SZ, SZ]),
    "vmlm_gemm_nt_bf16": (I, [P, P, P, SZ, SZ, SZ]),
    "vmlm_gemm_nt": (I, [P, P, P, SZ, SZ, SZ, B]),
    "vmlm_gemm": (I, [P, P, P, SZ, SZ, SZ, B]),
    "vmlm_rmsnorm": (I, [P, P, P, SZ, SZ, F]),
    "vmlm_softmax": (I, [P, SZ, SZ, B]),
    "vmlm_act": (I, [P, SZ, U16]),
    "vmlm_ew_op": (I, [P, P, P, SZ, U8]),
    "vmlm_scale": (I, [P, P, SZ, F]),
    "vmlm_rope": (I, [P, P, SZ, SZ, F, U16]),
    "vmlm_emb_bf16": (I, [P, P, SZ, SZ, F]),
    "vmlm_emb_f32": (I, [P, P, SZ, SZ, F]),
    "vmlm_topk_idx": (I, [P, SZ, SZ, P]),
    "vmlm_b1_forward": (I, [C.POINTER(SparseConnW), P, P, C.POINTER(SZ)]),
    "vmlm_b1_forward_t8": (I, [C.POINTER(SparseConnW), P, SZ, SZ, P, C.POINTER(SZ)]),
    "vmlm_b1_backward": (I, [C.POINTER(SparseConnW), P, P, P, C.POINTER(SZ)]),
    "vmlm_b1_backward_dx": (I, [C.POINTER(SparseConnW), P, P, C.POINTER(SZ)]),
    "vmlm_b1_backward_fused": (I, [C.POINTER(SparseConnW), P, P, P, P, C.POINTER(SZ)]),
    "vmlm_b1_backward_t8": (I, [P, P, P, P, SZ, SZ, SZ, P, P]),
    "vmlm_transpose_t8": (I, [P, SZ, SZ, P, SZ]),
    "vmlm_transpose_t8_back": (I, [P, SZ, SZ, P, SZ, SZ]),
    "vmlm_layernorm": (I, [P, P, P, SZ, SZ, F]),
    "vmlm_outer": (I, [P, P, P, SZ, SZ, F]),
    "vmlm_bias": (I, [P, P, SZ, SZ]),
    "vmlm_jit_gemm_nt": (I, [P, P, P, U64]),
    "vmlm_jit_act": (I, [P, SZ, U64]),
    "vmlm_jit_ewadd": (I, [P, P, P, SZ]),
    "vmlm_jit_ewmul": (I, [P, P, P, SZ]),
    "vmlm_jit_ewsub": (I, [P, P, P, SZ]),
    "vmlm_jit_ewdiv": (I, [P, P, P, SZ]),
    "vmlm_jit_bias": (I, [P, P, SZ, SZ]),
    "vmlm_jit_ln": (I, [P, P, P, U64, U64]),
    "vmlm_jit_softmax": (I, [P, U64, U64]),
    "vmlm_jit_outer": (I, [P, P, P, U64]),
    "vmlm_attention_prefill": (I, [P, P, P, P, SZ, SZ, SZ, F, U16, F, B]),
    "vmlm_attention_decode": (I, [P, P, P, P, P, P, SZ, SZ, SZ, SZ, F, F]),
    "vmlm_attention_decode_split": (I, [P, P, P, P, P, P, SZ, SZ, SZ, SZ, F, F, I]),
    # layer 2
    "vmlm_hip_gemm_nt_int8": (I, [P, P, P, P, SZ, SZ, SZ, P]),
    "vmlm_hip_gemm_nt_int8_noalloc": (I, [P, P, P, P, SZ, SZ, SZ, P]),
    "vmlm_hip_gemm_nt_bf16": (I, [P, P, P, SZ, SZ, SZ, P]),
    "vmlm_hip_gemm_nt_bf16bf16": (I, [P, P, P, SZ, SZ, SZ, P]),
    "vmlm_hip_gemm_nt": (I, [P, P, P, SZ, SZ, SZ, B, P]),
    "vmlm_hip_gemm": (I, [P, P, P, SZ, SZ, SZ, B, P]),
    "vmlm_hip_rmsnorm": (I, [P, P, P, SZ, SZ, F, P]),
    "vmlm_hip_softmax": (I, [P, SZ, SZ, B, P]),
    "vmlm_hip_act": (I, [P, SZ, U16, P]),
    "vmlm_hip_ew_op": (I, [P, P, P, SZ, U8, P]),
    "vmlm_hip_scale": (I, [P, P, SZ, F, P]),
    "vmlm_hip_rope": (I, [P, P, SZ, SZ, F, U16, P]),
    "vmlm_hip_emb_bf16": (I, [P, P, SZ, SZ, P, P]),
    "vmlm_hip_topk_idx": (I, [P, SZ, SZ, P, P]),
    "vmlm_hip_check_guards": (I, []),
    "vmlm_hip_b1_forward": (I, [C.POINTER(SparseConnW), P, P, SZ, P]),
    "vmlm_hip_b1_forward_t8": (I, [C.POINTER(SparseConnW), P, SZ, SZ, P, P]),
    "vmlm_hip_b1_backward_fused": (I, [C.POINTER(SparseConnW), P, P, P, P, P]),
    "vmlm_hip_b1_backward_t8": (I, [P, P, P, P, SZ, SZ, SZ, P, P, P]),
    "vmlm_hip_transpose_t8": (I, [P, SZ, SZ, P, SZ, P]),
    "vmlm_hip_transpose_t8_back": (I, [P, SZ, SZ, P, SZ, SZ, P]),
    "vmlm_hip_layernorm": (I, [P, P, P, SZ, SZ, F, P]),
    "vmlm_hip_outer": (I, [P, P, P, SZ, SZ, F, P]),
    "vmlm_hip_bias": (I, [P, P, SZ, SZ, P]),
    "vmlm_hip_attention_prefill": (I, [P, P, P, P, SZ, SZ, SZ, F, U16, F, B, P]),
    "vmlm_hip_attention_decode": (I, [P, P, P, P, P, P, SZ, SZ, SZ, SZ, F, F, P]),
    "vmlm_hip_attention_decode_split": (I, [P, P, P, P, P, P, SZ, SZ, SZ, SZ, F, F, I, P]),
    # layer 3
    "vmlm_decoder_create": (I, [C.POINTER(DecoderCfg), C.POINTER(P)]),
    "vmlm_decoder_destroy": (I, [P]),
    "vmlm_decoder_load_layer": (I, [P, U32] + [P] * 16),
    "vmlm_decoder_load_globals": (I, [P, P, P, P]),
    "vmlm_decoder_prefill": (I, [P, P, U32, P, P]),
    "vmlm_decoder_decode": (I, [P, U32, P, P]),
    "vmlm_decoder_position": (I, [P, C.POINTER(U32)]),
    "vmlm_decoder_set_graph": (I, [P, I]),
    "vmlm_decoder_stream": (P, [P]),
    "vmlm_decoder_set_fused": (I, [P, I]),
    "vmlm_decoder_fused": (I, [P]),
    "vmlm_decoder_set_program": (I, [P, I]),
    "vmlm_decoder_program": (I, [P]),
    "vmlm_decoder_time_gemv": (I, [P, I, U32, C.POINTER(F), C.POINTER(C.c_double)]),
    "vmlm_b1_stack_forward": (I, [C.POINTER(SparseConnW), U32, P, P, SZ, U16, P]),
    "vmlm_b1_stack_create": (I, [C.POINTER(SparseConnW), U32, P, C.POINTER(C.c_void_p)]),
    "vmlm_b1_stack_run": (I, [P, P, P, SZ, U16, P]),
    "vmlm_b1_stack_destroy": (I, [P]),
    "vmlm_vm_load": (I, [C.c_char_p, SZ, P, SZ, C.POINTER(P)]),
    "vmlm_vm_destroy": (I, [P]),
    "vmlm_vm_run": (I, [P]),
    "vmlm_vm_find_slot": (I, [P, C.c_char_p, C.POINTER(U32)]),
    "vmlm_vm_slot_info": (I, [P, U32, C.POINTER(P), C.POINTER(U32), C.POINTER(U32),
                              C.POINTER(U8)]),
    "vmlm_vm_write_slot": (I, [P, U32, P, SZ]),
    "vmlm_vm_read_slot": (I, [P, U32, P, SZ]),
    "vmlm_vm_output": (I, [P, P, SZ, C.POINTER(SZ)]),
    "vmlm_vm_clear_output": (I, [P]),
    "vmlm_vm_stream": (P, [P]),
    "vmlm_vm_pool_uploads": (I, [C.POINTER(SZ)]),
    "vmlm_vm_swizzled_consts": (I, [P, C.POINTER(SZ)]),
    "vmlm_vm_fused_runs": (I, [P, C.POINTER(SZ)]),
    "vmlm_vm_fused_opcodes": (I, [P, C.POINTER(SZ)]),
    "vmlm_vm_set_graphs": (I, [P, I]),
    "vmlm_vm_graph_segments": (I, [P, C.POINTER(SZ)]),
    "vmlm_hip_backend": (P, []),
    "vmlm_backend_dot256": (F, [P, P, SZ]),
    "vmlm_backend_axpy256": (None, [P, P, F, SZ]),
    "vmlm_backend_add256": (None, [P, P, SZ]),
    "vmlm_backend_max256": (F, [P, SZ]),
    "vmlm_backend_sum256": (F, [P, SZ]),
    "vmlm_backend_scale_mul": (None, [P, P, F, SZ]),
    "vmlm_hip_kernel_table": (P, []),
}


def declare(L: C.CDLL) -> None:
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)  # AttributeError = missing export: fail loudly
        fn.restype = res
        fn.argtypes = args

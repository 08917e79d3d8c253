"""ctypes binding of include/hayai_hip.h (the same binding a Rust/C caller writes).

Loading fails loudly: there is no CPU fallback anywhere in this package.  If the library
has not been built, :class:`LibraryMissing` tells the caller to run ``python -m
hayai_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhayai_hip.so")

HH_OK = 0
STATUS_NAMES = {
    0: "HH_OK",
    1: "HH_ERR_NO_DEVICE",
    2: "HH_ERR_INVALID",
    3: "HH_ERR_KERNEL_MISSING",
    4: "HH_ERR_RUNTIME",
    5: "HH_ERR_OUT_OF_MEMORY",
    6: "HH_ERR_UNSUPPORTED_DEVICE",
    7: "HH_ERR_IO",
    8: "HH_ERR_NOT_FOUND",
}

class GgufInfo(C.Structure):
    _fields_ = [
        ("version", C.c_uint32),
        ("io_uring", C.c_uint32),
        ("o_direct", C.c_uint32),
        ("pad", C.c_uint32),
        ("alignment", C.c_uint64),
        ("data_offset", C.c_uint64),
        ("header_bytes", C.c_uint64),
        ("n_tensors", C.c_uint64),
        ("n_metadata", C.c_uint64),
        ("file_size", C.c_uint64),
    ]


class GgufTensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("n_dims", C.c_uint32),
        ("type", C.c_uint32),
        ("dims", C.c_uint64 * 4),
        ("offset", C.c_uint64),
        ("abs_offset", C.c_uint64),
        ("nbytes", C.c_uint64),
    ]


class LayerPack(C.Structure):
    _fields_ = [
        ("off", C.c_size_t * 8),
        ("len", C.c_size_t * 8),
        ("type", C.c_uint32 * 8),
        ("cols", C.c_uint64 * 8),
        ("rows", C.c_uint64 * 8),
        ("total", C.c_size_t),
        ("fused_gate_up", C.c_int32),
        ("pad", C.c_int32),
    ]


# Every symbol include/hayai_hip.h declares, with (restype, argtypes).
P = C.c_void_p
SZ = C.c_size_t
I = C.c_int
ST = C.c_int
PP = C.POINTER(C.c_void_p)


class DeviceInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("arch", C.c_char * 64),
        ("device_index", C.c_int),
        ("compute_units", C.c_int),
        ("wavefront_size", C.c_int),
        ("clock_khz", C.c_int),
        ("memory_clock_khz", C.c_int),
        ("memory_bus_width", C.c_int),
        ("total_mem", C.c_size_t),
        ("lds_per_block", C.c_size_t),
        ("l2_bytes", C.c_size_t),
    ]


class FfnDesc(C.Structure):
    _fields_ = [
        ("type_gate", C.c_int),
        ("type_up", C.c_int),
        ("type_down", C.c_int),
        ("act", C.c_int),
        ("d_model", C.c_size_t),
        ("d_ff", C.c_size_t),
        ("gate_off", C.c_size_t),
        ("up_off", C.c_size_t),
        ("down_off", C.c_size_t),
    ]


class MoeDesc(C.Structure):
    _fields_ = [
        ("type", C.c_int),
        ("act", C.c_int),
        ("d_model", C.c_size_t),
        ("d_ff", C.c_size_t),
        ("n_experts", C.c_size_t),
        ("top_k", C.c_size_t),
        ("expert_stride", C.c_size_t),
        ("gate_off", C.c_size_t),
        ("up_off", C.c_size_t),
        ("down_off", C.c_size_t),
        ("n_group", C.c_size_t),
        ("topk_group", C.c_size_t),
        ("gating", C.c_int),
        ("norm_topk_prob", C.c_int),
        ("routed_scaling_factor", C.c_float),
        ("shared_d_ff", C.c_size_t),
        ("shared_gate_off", C.c_size_t),
        ("shared_up_off", C.c_size_t),
        ("shared_down_off", C.c_size_t),
    ]


SIGNATURES = {
    "hh_gguf_open": (ST, [C.c_char_p, PP]),
    "hh_gguf_close": (None, [P]),
    "hh_gguf_header": (ST, [P, C.POINTER(GgufInfo)]),
    "hh_gguf_tensor_at": (ST, [P, C.c_uint64, C.POINTER(GgufTensor)]),
    "hh_gguf_find": (ST, [P, C.c_char_p, C.POINTER(GgufTensor)]),
    "hh_gguf_meta_u32": (ST, [P, C.c_char_p, C.POINTER(C.c_uint32)]),
    "hh_gguf_meta_u64": (ST, [P, C.c_char_p, C.POINTER(C.c_uint64)]),
    "hh_gguf_meta_f32": (ST, [P, C.c_char_p, C.POINTER(C.c_float)]),
    "hh_gguf_meta_str": (ST, [P, C.c_char_p, C.POINTER(C.c_char_p), C.POINTER(SZ)]),
    "hh_tensor_nbytes": (ST, [C.c_uint32, C.POINTER(C.c_uint64), C.c_uint32, C.POINTER(C.c_uint64)]),
    "hh_gguf_layer_pack": (ST, [P, SZ, C.POINTER(LayerPack)]),
    "hh_gguf_load_layer_pack": (ST, [P, SZ, P, SZ, C.POINTER(LayerPack)]),
    "hh_gguf_read_tensor": (ST, [P, C.c_char_p, P, SZ]),
    "hh_abi_version": (C.c_int, []),
    "hh_last_error": (C.c_char_p, []),
    "hh_status_name": (C.c_char_p, [ST]),
    "hh_row_bytes": (ST, [I, SZ, C.POINTER(SZ)]),
    "hh_validate_gemv_shape": (ST, [I, SZ, SZ]),
    "hh_validate_gemv_weights": (ST, [I, SZ, SZ, SZ]),
    "hh_device_count": (ST, [C.POINTER(C.c_int)]),
    "hh_engine_create": (ST, [I, PP]),
    "hh_engine_destroy": (None, [P]),
    "hh_engine_info": (ST, [P, C.POINTER(DeviceInfo)]),
    "hh_engine_sync": (ST, [P]),
    "hh_engine_ffn_calls": (C.c_uint64, [P]),
    "hh_buf_alloc": (ST, [P, SZ, I, PP]),
    "hh_buf_free": (None, [P]),
    "hh_buf_size": (SZ, [P]),
    "hh_buf_kind": (C.c_int, [P]),
    "hh_buf_host_ptr": (P, [P]),
    "hh_buf_write": (ST, [P, P, SZ, P, SZ]),
    "hh_buf_read": (ST, [P, P, SZ, P, SZ]),
    "hh_buf_copy": (ST, [P, P, SZ, P, SZ, SZ]),
    "hh_buf_fill": (ST, [P, P, SZ, C.c_uint8, SZ]),
    "hh_gemv": (ST, [P, I, SZ, SZ, P, SZ, P, P]),
    "hh_gemv_bound": (ST, [P, I, SZ, SZ, P, SZ, P, P]),
    "hh_gemv_begin": (ST, [P, I, SZ, SZ, P, SZ, P, PP]),
    "hh_pending_wait": (ST, [P, P, SZ]),
    "hh_pending_destroy": (None, [P]),
    "hh_gemv_dev": (ST, [P, I, SZ, SZ, P, SZ, P, SZ, P, SZ]),
    "hh_dequant_dev": (ST, [P, I, P, SZ, SZ, P, SZ]),
    "hh_lut_gemv": (ST, [P, SZ, SZ, P, SZ, P, P, P]),
    "hh_lut_gemv_dev": (ST, [P, SZ, SZ, P, SZ, P, SZ, P, SZ, P, SZ]),
    "hh_ffn": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, P]),
    "hh_ffn_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ, P, SZ]),
    "hh_ffn_dev_noalloc": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ, P, SZ]),
    "hh_ffn_block_begin_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ, C.c_float, P, SZ]),
    "hh_ffn_block_finish_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ, P, SZ]),
    "hh_ffn_block_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ, C.c_float, P, SZ, P, SZ]),
    "hh_ffn_block_stack_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, SZ, SZ, P, SZ, SZ, C.c_float, P, SZ, P, SZ]),
    "hh_gemv_batched": (ST, [P, I, SZ, SZ, P, SZ, P, P, SZ]),
    "hh_gemv_batched_dev": (ST, [P, I, SZ, SZ, P, SZ, P, SZ, SZ, P, SZ]),
    "hh_ffn_batched_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ, SZ, P, SZ]),
    "hh_ffn_batched": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, P, SZ]),
    "hh_ffn_begin_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ]),
    "hh_ffn_finish_dev": (ST, [P, C.POINTER(FfnDesc), P, SZ, P, SZ]),
    "hh_gateup_dev": (ST, [P, I, I, SZ, SZ, P, SZ, P, SZ, P, SZ, P, SZ, I]),
    "hh_route_experts_dev": (ST, [P, C.POINTER(MoeDesc), P, SZ, P, SZ, SZ, P, SZ, P, SZ]),
    "hh_route_experts": (ST, [P, C.POINTER(MoeDesc), P, P, SZ, P, P]),
    "hh_moe_ffn_dev": (ST, [P, C.POINTER(MoeDesc), P, SZ, P, SZ, SZ, P, SZ, P, SZ, P, SZ]),
    "hh_moe_dev": (ST, [P, C.POINTER(MoeDesc), P, SZ, P, SZ, P, SZ, P, SZ, SZ, P, SZ]),
    "hh_streamer_create": (ST, [P, SZ, SZ, SZ, PP]),
    "hh_streamer_destroy": (None, [P]),
    "hh_streamer_slot_for": (ST, [P, SZ, C.POINTER(SZ)]),
    "hh_streamer_weight_offset": (ST, [P, SZ, SZ, C.POINTER(SZ)]),
    "hh_streamer_host_slot": (ST, [P, SZ, PP]),
    "hh_streamer_dma": (ST, [P, SZ, SZ, SZ]),
    "hh_streamer_bind": (ST, [P, SZ, PP, C.POINTER(SZ)]),
    "hh_event_create": (ST, [P, PP]),
    "hh_event_destroy": (None, [P]),
    "hh_event_record": (ST, [P, P]),
    "hh_event_elapsed_ms": (ST, [P, P, C.POINTER(C.c_float)]),
    "hh_graph_begin": (ST, [P]),
    "hh_graph_end": (ST, [P, PP]),
    "hh_graph_launch": (ST, [P]),
    "hh_graph_destroy": (None, [P]),
    "hh_synth_weights_dev": (ST, [P, I, P, SZ, SZ, C.c_uint64, C.c_float, C.c_float]),
}


class LibraryMissing(RuntimeError):
    pass


_lib = None


def load() -> C.CDLL:
    """Load libhayai_hip.so (in-tree) and declare every ABI symbol."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m hayai_amd.build` (the HIP library is required, "
            "there is no CPU fallback)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError = a header symbol the library lacks
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib

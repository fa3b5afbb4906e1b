"""Loads libifx_qgemm.so (the HIP kernels behind include/ifx_qgemm.h) with
ctypes and declares every exported C entry point.

There is no fallback: if the library is missing this raises, so nothing can
silently run another implementation in its place.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libifx_qgemm.so")

# Every symbol include/ifx_qgemm.h declares, with its ctypes signature.
_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
SIGNATURES = {
    "ifx_q8_1_quantize_f32": ([_vp, _vp, _i32, _i32, _vp], _i32),
    "ifx_q8_1_quantize_f16": ([_vp, _vp, _i32, _i32, _vp], _i32),
    "ifx_rmsnorm_quantize_q8_1": ([_vp, _i32, _vp, _vp, _i32, _i32, ctypes.c_float, _vp], _i32),
    "ifx_silu_mul_quantize_q8_1": ([_vp, _vp, _i32, _vp, _i32, _i32, _vp], _i32),
    "ifx_quantize_rows_symmetric": ([_vp, _i32, _vp, _vp, _i32, _i32, _vp], _i32),
    "ifx_silu_mul_quantize_rows_symmetric": ([_vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp], _i32),
    "ifx_qgemv_packed": ([_i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp], _i32),
    "ifx_qgemv": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp], _i32),
    "ifx_qgemv_grouped": ([_i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp], _i32),
    "ifx_qgemv_grouped_rmsnorm": ([_i32, _i32, _vp, _vp, _vp, _vp, _i32, _vp, ctypes.c_float, _i32, _i32, _i32, _i32, _vp], _i32),
    "ifx_qgemm_prefill_workspace_bytes": ([_i32, _i32, _i32, _i32], _i64),
    "ifx_qgemm_prefill_ws": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _i64, _vp],
                             _i32),
    "ifx_qgemv_gate_up_silu": ([_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp], _i32),
    "ifx_qgemv_gate_up_silu_ws": ([_i32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _i64,
                                   _vp], _i32),
    "ifx_qgemv_gate_up_silu_workspace_bytes": ([_i32, _i32, _i32, _i32], _i64),
    "ifx_qgemv_gate_up_silu_rmsnorm": ([_i32, _vp, _vp, _vp, _i32, _vp, ctypes.c_float, _vp, _i32, _vp, _i32,
                                        _i32, _i32, _vp], _i32),
    "ifx_qgemm_prefill_noalloc": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp], _i32),
    "ifx_qgemm_prefill_ordered_workspace_bytes": ([_i32, _i32, _i32, _i32, _i32], _i64),
    "ifx_qgemm_prefill_ordered": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _i64,
                                   _vp], _i32),
    "ifx_qgemm_prefill": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp], _i32),
    "ifx_qgemm_prefill_kernel": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _vp], _i32),
    "ifx_repacked_bytes": ([_i32, _i64, _i32], _i64),
    "ifx_repack": ([_i32, _vp, _vp, _i64, _i32, _vp], _i32),
    "ifx_tiled_bytes": ([_i32, _i64, _i32], _i64),
    "ifx_qgemv_ws": ([_i32, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _i64, _vp], _i32),
    "ifx_qgemv_grouped_ws": ([_i32, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _i64,
                              _vp], _i32),
    "ifx_qgemv_workspace_bytes": ([_i32, _i32, _vp, _i32, _i32, _i32], _i64),
    "ifx_repack_tiled": ([_i32, _vp, _vp, _i64, _i32, _vp], _i32),
    "ifx_mmq_layout_bytes": ([_i32, _i64, _i32], _i64),
    "ifx_mmq_layout_rows_offset": ([_i32, _i64, _i32], _i64),
    "ifx_mmq_layout_build": ([_i32, _vp, _vp, _i64, _i32, _vp], _i32),
    "ifx_mmq_layout_ws_offset": ([_i32, _i64, _i32], _i64),
    "ifx_qgemv_mmq": ([_i32, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp], _i32),
    "ifx_dequantize": ([_i32, _vp, _vp, _i32, _i64, _i32, _vp], _i32),
    "ifx_kernel_family": ([_i32, _i32, _i32, _i32], _i32),
    "ifx_launch_log_begin": ([_i32], None),
    "ifx_launch_log_end": ([], ctypes.c_char_p),
    "ifx_supports": ([_i32, _i32, _i32, _i32], _i32),
    "ifx_block_bytes": ([_i32], _i32),
    "ifx_block_elems": ([_i32], _i32),
    "ifx_status_string": ([_i32], ctypes.c_char_p),
}


class GgufTensor(ctypes.Structure):
    """ifx_gguf_tensor (include/ifx_gguf.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("shape", ctypes.c_int64 * 8), ("offset", ctypes.c_uint64),
                ("byte_size", ctypes.c_uint64), ("host_data", ctypes.c_void_p)]


# Every symbol include/ifx_gguf.h declares.
_u32, _u64, _cp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_char_p
_pp = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES.update({
    "ifx_gguf_open": ([_cp, _pp], _i32),
    "ifx_gguf_close": ([_vp], None),
    "ifx_gguf_version": ([_vp], _u32),
    "ifx_gguf_alignment": ([_vp], _u64),
    "ifx_gguf_data_offset": ([_vp], _u64),
    "ifx_gguf_n_tensors": ([_vp], _i64),
    "ifx_gguf_n_kv": ([_vp], _i64),
    "ifx_gguf_tensor_info": ([_vp, _i64, ctypes.POINTER(GgufTensor)], _i32),
    "ifx_gguf_find": ([_vp, _cp], _i64),
    "ifx_gguf_kv_key": ([_vp, _i64, ctypes.POINTER(_cp), ctypes.POINTER(_i32)], _i32),
    "ifx_gguf_get_int": ([_vp, _cp, ctypes.POINTER(_i64)], _i32),
    "ifx_gguf_get_float": ([_vp, _cp, ctypes.POINTER(ctypes.c_double)], _i32),
    "ifx_gguf_get_string": ([_vp, _cp, _pp, ctypes.POINTER(_u64)], _i32),
    "ifx_gguf_get_array": ([_vp, _cp, ctypes.POINTER(_i32), ctypes.POINTER(_u64)], _i32),
    "ifx_gguf_get_array_string": ([_vp, _cp, _u64, _pp, ctypes.POINTER(_u64)], _i32),
    "ifx_gguf_get_array_data": ([_vp, _cp, _pp, ctypes.POINTER(_i32), ctypes.POINTER(_u64)], _i32),
    "ifx_gguf_device_bytes": ([_vp, _u64], _u64),
    "ifx_gguf_upload": ([_vp, _vp, _u64, _u64, ctypes.POINTER(_u64), _vp], _i32),
    "ifx_gguf_tensor_bytes": ([_i32, ctypes.POINTER(_i64), _i32], _u64),
    "ifx_gguf_type_name": ([_i32], _cp),
    "ifx_gguf_parse_name": ([_cp, ctypes.POINTER(_i32), _cp, _u64, _cp, _u64], _i32),
    "ifx_gguf_status_string": ([_i32], _cp),
})

_lib = None


class IfxError(RuntimeError):
    pass


def load():
    """Returns the loaded library; raises IfxError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise IfxError(
                "libifx_qgemm.so is not built (run `python -m inferflux_amd.build`); "
                "the quantized GEMV/GEMM path has no other implementation")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib

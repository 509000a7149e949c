"""ctypes binding of the engine's C ABI (include/jax4j_mi355x.h).

The shared library is built in-tree (``jax4j_amd/lib/libjax4j_mi355x.so``). There is no
fallback: if the library is missing, loading raises, so a GPU run can never silently
execute anything but the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("JAX4J_MI355X_LIB", Path(__file__).resolve().parent / "lib" / "libjax4j_mi355x.so"))

J4Q_OK = 0
J4Q_EINVAL = 1
J4Q_EUNSUPPORTED = 2
J4Q_ENODEV = 3
J4Q_EHIP = 4
J4Q_ENOMEM = 5
J4Q_EHANDLE = 6

KIND_QUANT = 1
KIND_F32 = 2
KIND_BF16 = 3
KIND_I8 = 4

GEMM_INT8 = 0
GEMM_BF16 = 1
# j4q_gemv_policy
GEMV_MATRIX_CORES = 0
GEMV_FP32 = 1


class DeviceProps(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("arch", C.c_char * 64),
        ("device", C.c_int32),
        ("compute_units", C.c_int32),
        ("max_clock_khz", C.c_int32),
        ("l2_bytes", C.c_int32),
        ("hbm_bytes", C.c_uint64),
    ]


class BufferDesc(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("quant_type", C.c_int32),
        ("rank", C.c_int32),
        ("reserved", C.c_int32),
        ("dims", C.c_int64 * 2),
        ("bytes", C.c_uint64),
        ("device_ptr", C.c_void_p),
    ]


class GgufInfo(C.Structure):
    _fields_ = [
        ("version", C.c_uint32),
        ("reserved", C.c_uint32),
        ("tensor_count", C.c_int64),
        ("metadata_count", C.c_int64),
        ("alignment", C.c_uint64),
        ("data_offset", C.c_uint64),
        ("file_bytes", C.c_uint64),
    ]


class GgufTensor(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("type_id", C.c_int32),
        ("n_dims", C.c_int32),
        ("dims", C.c_int64 * 4),
        ("offset", C.c_uint64),
        ("nbytes", C.c_uint64),
    ]


class DecodeLayer(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("q", "k", "v", "o", "gate", "up", "down")]


class DecodeIO(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")]


class DecodePlanDesc(C.Structure):
    _fields_ = [
        ("layers", C.c_int32),
        ("graph", C.c_int32),
        ("batch", C.c_int64),
        ("d_model", C.c_int64),
        ("qkv_rows", C.c_int64),
        ("o_cols", C.c_int64),
        ("ffn", C.c_int64),
        ("vocab", C.c_int64),
        ("gemvs_per_step", C.c_int64),
        ("weight_bytes", C.c_uint64),
        ("plan_bytes", C.c_uint64),
    ]


_i32, _i64, _u64, _vp = C.c_int32, C.c_int64, C.c_uint64, C.c_void_p
_buf = C.c_uint64
_pbuf = C.POINTER(C.c_uint64)

# name -> (argtypes); every function returns int (status) unless listed in _RESTYPES.
SIGNATURES = {
    "j4q_abi_version": [],
    "j4q_probe": [],
    "j4q_init": [C.c_int],
    "j4q_last_error": [],
    "j4q_device_info": [C.POINTER(DeviceProps)],
    "j4q_sync": [],
    "j4q_stream": [C.POINTER(C.c_void_p)],
    "j4q_quant_type_info": [C.c_int, C.POINTER(_i32), C.POINTER(_i32)],
    "j4q_quant_byte_size": [C.c_int, _i64, C.POINTER(_u64)],
    "j4q_supported_quant_types": [C.POINTER(_i32), _i32, C.POINTER(_i32)],
    "j4q_upload_quantized": [C.c_int, _vp, _u64, _i64, _i64, _pbuf],
    "j4q_upload_quantized_device": [C.c_int, _vp, _u64, _i64, _i64, _pbuf],
    "j4q_export_quantized": [_buf, _vp, _u64],
    "j4q_concat_rows": [_pbuf, _i32, _pbuf],
    "j4q_upload_f32": [_vp, _i32, C.POINTER(_i64), _pbuf],
    "j4q_upload_bf16": [_vp, _i32, C.POINTER(_i64), _pbuf],
    "j4q_download_f32": [_buf, _vp, _i64],
    "j4q_download_bytes": [_buf, _vp, _u64],
    "j4q_buffer_info": [_buf, C.POINTER(BufferDesc)],
    "j4q_release": [_buf],
    "j4q_buffer_stats": [C.POINTER(_i64), C.POINTER(_u64)],
    "j4q_quant_matvec": [_buf, _buf, _pbuf],
    "j4q_quant_matvec_add": [_buf, _buf, _buf, _pbuf],
    "j4q_quant_gather_row": [_buf, _i64, _pbuf],
    "j4q_quant_dequantize": [_buf, _pbuf],
    "j4q_set_gemv_policy": [C.c_int, C.POINTER(C.c_int)],
    "j4q_quantize_act": [_buf, _pbuf, _pbuf],
    "j4q_quant_matmul": [_buf, _buf, C.c_int, _pbuf],
    "j4q_quant_matvec_into": [_buf, _vp, _vp, _vp, _i64, _vp],
    "j4q_quant_matmul_into": [_buf, _vp, _i64, C.c_int, _vp, _vp, _vp, _vp],
    "j4q_quant_matmul_noalloc": [_buf, _vp, _i64, C.c_int, _vp, _vp],
    "j4q_quant_matmul_q8_into": [_buf, _vp, _vp, _i64, _vp, _vp],
    "j4q_synth_quant_host": [C.c_int, _u64, _i64, _i64, _vp, _u64],
    "j4q_synth_quant_device": [C.c_int, _u64, _i64, _i64, _vp, _u64, _vp],
    "j4q_synth_f32_host": [_u64, _i64, _vp],
    "j4q_synth_bf16_host": [_u64, _i64, _vp],
    "j4q_synth_f32_device": [_u64, _i64, _vp, _vp],
    "j4q_synth_bf16_device": [_u64, _i64, _vp, _vp],
    "j4q_decode_plan_create": [C.POINTER(DecodeLayer), _i32, _buf, _i64, C.POINTER(DecodeIO), C.POINTER(_u64)],
    "j4q_decode_plan_run": [_u64, _vp],
    "j4q_decode_plan_info": [_u64, C.POINTER(DecodePlanDesc)],
    "j4q_decode_plan_destroy": [_u64],
    "j4q_gguf_open": [C.c_char_p, C.POINTER(_u64)],
    "j4q_gguf_close": [_u64],
    "j4q_gguf_file_info": [_u64, C.POINTER(GgufInfo)],
    "j4q_gguf_tensor_info": [_u64, _i64, C.POINTER(GgufTensor)],
    "j4q_gguf_find_tensor": [_u64, C.c_char_p, C.POINTER(_i64)],
    "j4q_gguf_meta_key": [_u64, _i64, C.c_char_p, _i32, C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_u64)],
    "j4q_gguf_meta_scalar": [_u64, C.c_char_p, C.POINTER(_i32), _vp],
    "j4q_gguf_meta_string": [_u64, C.c_char_p, C.c_char_p, _u64, C.POINTER(_u64)],
    "j4q_gguf_read_tensor": [_u64, _i64, _vp, _u64],
    "j4q_gguf_upload": [_u64, _i64, _pbuf],
    "j4q_spin": [C.c_uint32, _vp],
    "j4q_copy": [_vp, _vp, _u64, _vp],
    "j4q_stream_read": [_vp, _u64, _vp, _i32, _i32, _vp],
    "j4q_gemv_trace": [_vp, _i64],
}
_RESTYPES = {"j4q_last_error": C.c_char_p}

_lib: C.CDLL | None = None


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def load() -> C.CDLL:
    """Load the engine library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"jax4j MI355X engine library not found at {LIB_PATH}; build it with "
            "`python -m jax4j_amd.build` (or __graft_entry__.build())"
        )
    lib = C.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, C.c_int)
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().j4q_last_error()
    return msg.decode() if msg else ""

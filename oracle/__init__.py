"""CPU oracle for the GGUF quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker or the timed CPU baseline; the engine
(``jax4j_amd``) never uses it. It wraps ``libquantref.so``, the C restatement in
``quant_ref.c`` (each function there cites the reference file:line it follows).

Parity status of each function (what pins it; see tests/test_oracle.py):
- ref_half_to_float: exhaustive 65,536-pattern check against numpy.float16.
- ref_q4_0_multiply / ref_q4_0_gather: restated from CpuQ4Gemm.java; pinned by hand-built
  known answers, the one-hot column identity, an fp64 brute force and an independent numpy
  decoder. No golden vectors exist in the reference for this path.
- ref_q2_0_*: same checks as Q4_0 (CpuQ2Gemm.java).
- Q8_0 / Q4_K / Q6_K dequant: no reference arithmetic (ggml format spec only); pinned by
  hand-derived single-block known answers and an independent numpy decoder written from
  the published block layouts.
- ref_quantize_act, GEMM references: pinned by closed-form cases (constant blocks, zero
  blocks, exact powers of two) and by exact integer arithmetic checks in numpy.
- ref_matmul_f64: each row equals ref_matvec_f64 of its batch row bit for bit, and the
  whole product equals a numpy fp64 product of the decoded matrix within 1e-12.
- ref_gemm_f64 / ref_gemm_bf16w_f64 (any format): equal the Q8_0 entry points bit for bit
  on Q8_0, and a numpy fp64 product of the decoded (or bf16-rounded) weights within 1e-12.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libquantref.so"

Q4_0, Q8_0, Q4_K, Q6_K, Q2_0 = 2, 8, 12, 14, 42
GEOMETRY = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q2_0: (128, 34)}

_lib = None
_vp, _i64 = C.c_void_p, C.c_int64


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing at {LIB_PATH}; run `make -C oracle`")
        lib = C.CDLL(str(LIB_PATH))
        sig = {
            "ref_block_geometry": [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)],
            "ref_half_to_float": [C.c_uint32],
            "ref_half_to_float_array": [_vp, _vp, _i64],
            "ref_q4_0_multiply": [_vp, _vp, _vp, _i64, _i64],
            "ref_q4_0_gather": [_vp, _vp, _i64, _i64, _i64],
            "ref_q2_0_multiply": [_vp, _vp, _vp, _i64, _i64],
            "ref_q2_0_gather": [_vp, _vp, _i64, _i64, _i64],
            "ref_dequant_row": [C.c_int, _vp, _i64, _vp],
            "ref_matvec": [C.c_int, _vp, _i64, _i64, _vp, _vp],
            "ref_matvec_f64": [C.c_int, _vp, _i64, _i64, _vp, _vp],
            "ref_matmul_f64": [C.c_int, _vp, _i64, _i64, _vp, _i64, _vp],
            "ref_dequant_matrix": [C.c_int, _vp, _i64, _i64, _vp],
            "ref_f32_to_bf16": [C.c_float],
            "ref_bf16_to_f32": [C.c_uint16],
            "ref_quantize_act": [_vp, _i64, _i64, _vp, _vp],
            "ref_gemm_q8_int8_emulated": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
            "ref_gemm_q8_int8_emulated_ranges": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp],
            "ref_gemm_q8_f64": [_vp, _vp, _i64, _i64, _i64, _vp],
            "ref_gemm_f64": [C.c_int, _vp, _vp, _i64, _i64, _i64, _vp],
            "ref_gemm_bf16w_f64": [C.c_int, _vp, _vp, _i64, _i64, _i64, _vp],
            "ref_gemm_q8_bf16w_f64": [_vp, _vp, _i64, _i64, _i64, _vp],
        }
        res = {"ref_half_to_float": C.c_float, "ref_half_to_float_array": None, "ref_f32_to_bf16": C.c_uint16, "ref_bf16_to_f32": C.c_float}
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res.get(name, C.c_int)
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments")


def half_to_float(bits: int) -> float:
    return load().ref_half_to_float(bits)


def half_to_float_array(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    load().ref_half_to_float_array(_p(h), _p(out), h.size)
    return out


def matvec(qtype: int, blob: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """Float-accumulated reference GEMV (the reference's own loop for Q4_0 / Q2_0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    _ok(load().ref_matvec(qtype, _p(blob), rows, cols, _p(x), _p(y)), "matvec")
    return y


def matvec_f64(qtype: int, blob: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float64)
    _ok(load().ref_matvec_f64(qtype, _p(blob), rows, cols, _p(x), _p(y)), "matvec_f64")
    return y


def matmul_f64(qtype: int, blob: np.ndarray, rows: int, cols: int, xs: np.ndarray) -> np.ndarray:
    """matvec_f64 of every row of xs [B, cols] -> [B, rows]; row b equals matvec_f64(xs[b])."""
    xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1, cols)
    y = np.empty((xs.shape[0], rows), dtype=np.float64)
    _ok(load().ref_matmul_f64(qtype, _p(blob), rows, cols, _p(xs), xs.shape[0], _p(y)), "matmul_f64")
    return y


def q4_0_multiply(blob: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    _ok(load().ref_q4_0_multiply(_p(y), _p(x), _p(blob), rows, cols), "q4_0_multiply")
    return y


def gather_row(qtype: int, blob: np.ndarray, row: int, rows: int, cols: int) -> np.ndarray:
    be, bb = GEOMETRY[qtype]
    rb = cols // be * bb
    if not 0 <= row < rows:
        raise ValueError("row out of range")
    out = np.empty(cols, dtype=np.float32)
    seg = np.ascontiguousarray(blob[row * rb:(row + 1) * rb])
    _ok(load().ref_dequant_row(qtype, _p(seg), cols, _p(out)), "dequant_row")
    return out


def dequant_matrix(qtype: int, blob: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    _ok(load().ref_dequant_matrix(qtype, _p(blob), rows, cols, _p(out)), "dequant_matrix")
    return out


def quantize_act(x_bf16: np.ndarray, m: int, k: int):
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    q = np.empty((m, k), dtype=np.int8)
    s = np.empty((m, k // 32), dtype=np.float32)
    _ok(load().ref_quantize_act(_p(x), m, k, _p(q), _p(s)), "quantize_act")
    return q, s


def gemm_int8_emulated(xq, xs, w_blob, m, n, k, ranges: int = 1, stage_blocks: int = 4) -> np.ndarray:
    """Emulated int8 GEMM; ranges > 1 cuts K into that many contiguous ranges of whole
    stages, folds each into its own partial and adds the partials in order."""
    y = np.empty((m, n), dtype=np.float32)
    _ok(load().ref_gemm_q8_int8_emulated_ranges(_p(np.ascontiguousarray(xq)), _p(np.ascontiguousarray(xs)), _p(w_blob), m, n,
                                                k, ranges, stage_blocks if ranges > 1 else 1, _p(y)), "gemm_int8")
    return y


def gemm_f64(x_bf16, w_blob, m, n, k, bf16_weights: bool = False, qtype: int = Q8_0) -> np.ndarray:
    """Y [m, n] = X_bf16 [m, k] . W^T in double for W of type `qtype` [n, k]: the exactly
    decoded weights, or with bf16_weights each fp32 weight rounded to bf16 first."""
    y = np.empty((m, n), dtype=np.float64)
    fn = load().ref_gemm_bf16w_f64 if bf16_weights else load().ref_gemm_f64
    _ok(fn(qtype, _p(np.ascontiguousarray(x_bf16, dtype=np.uint16)), _p(w_blob), m, n, k, _p(y)), "gemm_f64")
    return y


def gemm_q8_f64(x_bf16, w_blob, m, n, k, bf16_weights: bool = False) -> np.ndarray:
    """The Q8_0 entry points of the same two references."""
    y = np.empty((m, n), dtype=np.float64)
    fn = load().ref_gemm_q8_bf16w_f64 if bf16_weights else load().ref_gemm_q8_f64
    _ok(fn(_p(np.ascontiguousarray(x_bf16, dtype=np.uint16)), _p(w_blob), m, n, k, _p(y)), "gemm_q8_f64")
    return y

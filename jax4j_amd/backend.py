"""The MI355X quantized-matmul backend: a host-side mirror of the reference SPI over the C ABI.

``Mi355xBackend`` offers the reference's ``QuantizedOps`` capability
(``jax4j-core/.../tensor/spi/QuantizedOps.java:19-34``) plus the ``ComputeBackend`` members
this path needs (``name``, ``deviceType``, ``isAvailable``, ``priority``, ``upload``,
``download``, ``sync``, ``release``; ``spi/ComputeBackend.java:38-48, 87, 277-280``), with the
same argument meaning and error types. Every operation runs the engine's HIP kernels through
``libjax4j_mi355x.so``; nothing here computes on the CPU.

Engine-local extensions (no SPI counterpart): batched ``quant_matvec`` over x [B, K],
``quant_matmul`` (prefill GEMM, Q8_0 / Q4_0 / Q4_K / Q6_K weights x bf16 activations), ``quantize_act``,
``dequantize`` and ``export_quantized``.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import numpy as np

from . import _native as N
from .tensor import (
    Device,
    DeviceBuffer,
    DeviceType,
    DType,
    IllegalArgumentException,
    IllegalStateException,
    QuantType,
)

_ERRORS = {
    N.J4Q_EINVAL: IllegalArgumentException,
    N.J4Q_EUNSUPPORTED: IllegalArgumentException,
    N.J4Q_EHANDLE: IllegalArgumentException,
    N.J4Q_ENODEV: IllegalStateException,
}


def check(rc: int, op: str) -> None:
    """Raise the exception type the reference uses for a failing engine call."""
    if rc == N.J4Q_OK:
        return
    msg = N.last_error() or f"{op} failed (code {rc})"
    raise _ERRORS.get(rc, RuntimeError)(msg)


def _as_u8(blocks) -> np.ndarray:
    if isinstance(blocks, np.ndarray):
        return np.ascontiguousarray(blocks).reshape(-1).view(np.uint8)
    return np.frombuffer(memoryview(blocks).cast("B"), dtype=np.uint8)


class Mi355xBackend:
    """ComputeBackend + QuantizedOps for gfx950, selected by the name ``mi355x``."""

    NAME = "mi355x"
    PRIORITY = 60  # above RocmBackend's 50 (RocmBackend.java:443), below CUDA's 100

    def __init__(self, device: int = 0):
        self._device = device
        self._lock = threading.Lock()
        self._ready = False

    # ---- ComputeBackend identity (spi/ComputeBackend.java:38-46) -------------------------
    def name(self) -> str:
        return self.NAME

    def device_type(self) -> DeviceType:
        return DeviceType.ROCM

    def is_available(self) -> bool:
        """Never raises (HipRuntime.probe pattern, rocm/HipRuntime.java:145-158)."""
        try:
            return bool(N.load().j4q_probe())
        except Exception:
            return False

    def priority(self) -> int:
        return self.PRIORITY

    def _lib(self):
        lib = N.load()
        if not self._ready:
            with self._lock:
                if not self._ready:
                    check(lib.j4q_init(self._device), "init")
                    self._ready = True
        return lib

    def device_info(self) -> dict:
        props = N.DeviceProps()
        check(self._lib().j4q_device_info(C.byref(props)), "device_info")
        return {
            "name": props.name.decode(),
            "arch": props.arch.decode(),
            "device": props.device,
            "compute_units": props.compute_units,
            "max_clock_khz": props.max_clock_khz,
            "l2_bytes": props.l2_bytes,
            "hbm_bytes": props.hbm_bytes,
        }

    # ---- QuantizedOps (spi/QuantizedOps.java:19-34) --------------------------------------
    def supported_quant_types(self) -> set:
        ids = (C.c_int32 * 16)()
        n = C.c_int32()
        check(N.load().j4q_supported_quant_types(ids, 16, C.byref(n)), "supportedQuantTypes")
        return {QuantType.by_id(ids[i]) for i in range(n.value)}

    def upload_quantized(self, blocks, type: QuantType, logical_shape, device: Device | None = None) -> DeviceBuffer:
        """uploadQuantized (QuantizedOps.java:24). ``logical_shape`` = (rows, cols)."""
        shape = tuple(int(d) for d in logical_shape)
        if len(shape) != 2:
            raise IllegalArgumentException(f"uploadQuantized requires a rank-2 logical shape, got {shape}")
        self._check_device(device)
        data = _as_u8(blocks)
        out = C.c_uint64()
        check(
            self._lib().j4q_upload_quantized(
                type.id, data.ctypes.data_as(C.c_void_p), data.nbytes, shape[0], shape[1], C.byref(out)
            ),
            "uploadQuantized",
        )
        return DeviceBuffer(out.value, shape, DType.F32, Device.rocm(self._device), type)

    def upload_quantized_device(self, device_ptr: int, nbytes: int, type: QuantType, logical_shape) -> DeviceBuffer:
        """uploadQuantized for a GGUF blob already in device memory."""
        shape = tuple(int(d) for d in logical_shape)
        out = C.c_uint64()
        check(
            self._lib().j4q_upload_quantized_device(type.id, C.c_void_p(device_ptr), nbytes, shape[0], shape[1], C.byref(out)),
            "uploadQuantized",
        )
        return DeviceBuffer(out.value, shape, DType.F32, Device.rocm(self._device), type)

    def quant_matvec(self, weights: DeviceBuffer, x: DeviceBuffer) -> DeviceBuffer:
        """quantMatvec (QuantizedOps.java:27): y(rows) = W(rows, cols) . x(cols)."""
        out = C.c_uint64()
        check(self._lib().j4q_quant_matvec(weights.handle, x.handle, C.byref(out)), "quantMatvec")
        return self._dense_result(out.value, weights, x)

    def quant_matvec_add(self, weights: DeviceBuffer, x: DeviceBuffer, add: DeviceBuffer) -> DeviceBuffer:
        """quantMatvecAdd (QuantizedOps.java:30): y = W . x + add (add rounded separately)."""
        out = C.c_uint64()
        check(self._lib().j4q_quant_matvec_add(weights.handle, x.handle, add.handle, C.byref(out)), "quantMatvecAdd")
        return self._dense_result(out.value, weights, x)

    def quant_gather_row(self, weights: DeviceBuffer, row: int) -> DeviceBuffer:
        """quantGatherRow (QuantizedOps.java:33): one dequantized row, F32 [cols]."""
        out = C.c_uint64()
        check(self._lib().j4q_quant_gather_row(weights.handle, int(row), C.byref(out)), "quantGatherRow")
        return DeviceBuffer(out.value, (weights.shape[1],), DType.F32, weights.device)

    # ---- ComputeBackend data movement (spi/ComputeBackend.java:48, 87, 277, 280) ----------
    def upload(self, data, shape=None, dtype: DType = DType.F32, device: Device | None = None) -> DeviceBuffer:
        self._check_device(device)
        if dtype == DType.F32:
            arr = np.ascontiguousarray(np.asarray(data, dtype=np.float32))
            fn, elem = self._lib().j4q_upload_f32, 4
        elif dtype == DType.BF16:
            arr = np.ascontiguousarray(np.asarray(data, dtype=np.uint16))
            fn, elem = self._lib().j4q_upload_bf16, 2
        else:
            raise IllegalArgumentException(f"{self.NAME} upload supports F32 and BF16, got {dtype}")
        shape = tuple(int(d) for d in (arr.shape if shape is None else shape))
        if int(np.prod(shape, dtype=np.int64)) != arr.size:
            raise IllegalArgumentException(f"upload: {arr.size} values do not fill shape {shape}")
        dims = (C.c_int64 * 2)(*(list(shape) + [0] * (2 - len(shape))))
        out = C.c_uint64()
        check(fn(arr.ctypes.data_as(C.c_void_p), len(shape), dims, C.byref(out)), "upload")
        return DeviceBuffer(out.value, shape, dtype, Device.rocm(self._device))

    def download(self, buffer: DeviceBuffer) -> np.ndarray:
        """A fresh float32 copy of an F32 buffer (flat, like the reference's float[])."""
        if buffer.dtype != DType.F32 or buffer.quant_type is not None:
            return self.download_raw(buffer)
        out = np.empty(buffer.size(), dtype=np.float32)
        check(self._lib().j4q_download_f32(buffer.handle, out.ctypes.data_as(C.c_void_p), out.size), "download")
        return out

    def download_raw(self, buffer: DeviceBuffer) -> np.ndarray:
        dt = {DType.F32: np.float32, DType.BF16: np.uint16, DType.I8: np.int8}[buffer.dtype]
        out = np.empty(buffer.size(), dtype=dt)
        check(self._lib().j4q_download_bytes(buffer.handle, out.ctypes.data_as(C.c_void_p), out.nbytes), "download")
        return out

    def sync(self) -> None:
        check(self._lib().j4q_sync(), "sync")

    def release(self, buffer: DeviceBuffer) -> None:
        check(N.load().j4q_release(buffer.handle), "release")
        buffer.handle = 0

    # ---- engine-local extensions ----------------------------------------------------------
    def quant_matmul(self, weights: DeviceBuffer, x: DeviceBuffer, variant: str = "int8") -> DeviceBuffer:
        """Prefill GEMM Y[M, N] = X[M, K] . W^T for bf16 X: "int8" over Q8_0 W, "bf16" over
        Q8_0, Q4_0 (K % 128 == 0), Q4_K and Q6_K W (quantMatvec per row of X)."""
        v = {"int8": N.GEMM_INT8, "bf16": N.GEMM_BF16}.get(variant)
        if v is None:
            raise IllegalArgumentException(f"unknown GEMM variant {variant!r}")
        out = C.c_uint64()
        check(self._lib().j4q_quant_matmul(weights.handle, x.handle, v, C.byref(out)), "quantMatmul")
        return DeviceBuffer(out.value, (x.shape[0], weights.shape[0]), DType.F32, weights.device)

    def quantize_act(self, x: DeviceBuffer) -> tuple:
        q, s = C.c_uint64(), C.c_uint64()
        check(self._lib().j4q_quantize_act(x.handle, C.byref(q), C.byref(s)), "quantizeAct")
        m, k = x.shape
        return (
            DeviceBuffer(q.value, (m, k), DType.I8, x.device),
            DeviceBuffer(s.value, (m, k // 32), DType.F32, x.device),
        )

    def set_gemv_policy(self, policy: str) -> str:
        """Arithmetic of batched GEMV (engine-local): "matrix_cores" (default; launches of up
        to 16 batch rows, x as hi + lo fp16) or "fp32" (every row on the batch-1 kernel, equal
        bit for bit to quantMatvec of that row). Process-wide; returns the policy replaced."""
        names = {"matrix_cores": N.GEMV_MATRIX_CORES, "fp32": N.GEMV_FP32}
        if policy not in names:
            raise IllegalArgumentException(f"unknown GEMV policy {policy!r} (matrix_cores or fp32)")
        prev = C.c_int()
        # a process-wide setting of the library: no device needed
        check(N.load().j4q_set_gemv_policy(names[policy], C.byref(prev)), "setGemvPolicy")
        return {v: k for k, v in names.items()}[prev.value]

    def dequantize(self, weights: DeviceBuffer) -> DeviceBuffer:
        out = C.c_uint64()
        check(self._lib().j4q_quant_dequantize(weights.handle, C.byref(out)), "dequantize")
        return DeviceBuffer(out.value, tuple(weights.shape), DType.F32, weights.device)

    def concat_rows(self, parts) -> DeviceBuffer:
        """One quantized matrix holding the rows of ``parts`` in order (same type and cols):
        matrices that share an input run as one GEMV (engine-local; no SPI counterpart)."""
        parts = list(parts)
        if not parts or any(p.quant_type is None for p in parts):
            raise IllegalArgumentException("concat_rows needs quantized buffers")
        arr = (C.c_uint64 * len(parts))(*[p.handle for p in parts])
        out = C.c_uint64()
        check(self._lib().j4q_concat_rows(arr, len(parts), C.byref(out)), "concat_rows")
        rows = sum(p.shape[0] for p in parts)
        return DeviceBuffer(out.value, (rows, parts[0].shape[1]), DType.F32, Device.rocm(self._device), parts[0].quant_type)

    def export_quantized(self, weights: DeviceBuffer) -> np.ndarray:
        nbytes = weights.quant_type.byte_size_for(weights.shape[0] * weights.shape[1])
        out = np.empty(nbytes, dtype=np.uint8)
        check(self._lib().j4q_export_quantized(weights.handle, out.ctypes.data_as(C.c_void_p), nbytes), "export")
        return out

    def buffer_desc(self, buffer: DeviceBuffer) -> N.BufferDesc:
        d = N.BufferDesc()
        check(N.load().j4q_buffer_info(buffer.handle, C.byref(d)), "buffer_info")
        return d

    def buffer_stats(self) -> tuple:
        """(live buffer handles, device bytes they hold)."""
        n, b = C.c_int64(), C.c_uint64()
        check(self._lib().j4q_buffer_stats(C.byref(n), C.byref(b)), "buffer_stats")
        return n.value, b.value

    def stream(self) -> int:
        s = C.c_void_p()
        check(self._lib().j4q_stream(C.byref(s)), "stream")
        return s.value or 0

    def quant_matvec_into(self, weights: DeviceBuffer, x_ptr: int, add_ptr: int, y_ptr: int, batch: int = 1, stream: int = 0) -> None:
        """Stream-ordered GEMV on caller device memory; does not sync. A batched call over
        several column windows takes its partial-sum workspace from stream-ordered memory."""
        check(
            self._lib().j4q_quant_matvec_into(
                weights.handle, C.c_void_p(x_ptr), C.c_void_p(add_ptr or None), C.c_void_p(y_ptr), batch, C.c_void_p(stream or None)
            ),
            "quantMatvec_into",
        )

    def quant_matmul_into(self, weights: DeviceBuffer, x_ptr: int, m: int, variant: str, xq_ptr: int, xs_ptr: int, y_ptr: int, stream: int = 0) -> None:
        v = {"int8": N.GEMM_INT8, "bf16": N.GEMM_BF16}[variant]
        check(
            self._lib().j4q_quant_matmul_into(
                weights.handle, C.c_void_p(x_ptr), m, v, C.c_void_p(xq_ptr or None), C.c_void_p(xs_ptr or None),
                C.c_void_p(y_ptr), C.c_void_p(stream or None)
            ),
            "quantMatmul_into",
        )

    def decode_plan(self, layers, head, batch: int, io: dict) -> "DecodePlan":
        """The quantized matmuls of a decode step as one replayable plan (engine-local).

        ``layers``: per layer a dict of quantized buffers q, k, v, o, gate, up, down; ``head``:
        the output head or None; ``io``: device pointers h (residual stream, updated in place),
        x_o, x_down (inputs of o and down), qkv, gate_up (per-layer outputs) and logits.
        Per layer: qkv = [q|k|v].h; h' = o.x_o + h; gate_up = [gate|up].h'; h = down.x_down + h';
        finally logits = head.h.
        """
        arr = (N.DecodeLayer * len(layers))()
        for i, l in enumerate(layers):
            for k in ("q", "k", "v", "o", "gate", "up", "down"):
                setattr(arr[i], k, l[k].handle)
        cio = N.DecodeIO(**{k: C.c_void_p(io.get(k) or None) for k in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")})
        out = C.c_uint64()
        check(
            self._lib().j4q_decode_plan_create(arr, len(layers), head.handle if head else 0, batch, C.byref(cio), C.byref(out)),
            "decode plan",
        )
        return DecodePlan(self, out.value)

    # ---- helpers ---------------------------------------------------------------------------
    def _check_device(self, device: Device | None) -> None:
        if device is not None and (device.type != DeviceType.ROCM or device.index != self._device):
            raise IllegalArgumentException(f"{self.NAME} serves rocm:{self._device}, not {device}")

    def _dense_result(self, handle: int, weights: DeviceBuffer, x: DeviceBuffer) -> DeviceBuffer:
        rows, cols = weights.shape
        if x.size() == cols:
            shape = (rows,)
        else:
            shape = (x.shape[0], rows)
        return DeviceBuffer(handle, shape, DType.F32, weights.device)


class DecodePlan:
    """A decode step built once by ``Mi355xBackend.decode_plan`` (one captured HIP graph)."""

    def __init__(self, backend: Mi355xBackend, handle: int):
        self._be = backend
        self.handle = handle

    def run(self, stream: int = 0) -> None:
        """Enqueue one step on ``stream`` (0 = the engine stream); no synchronisation."""
        check(self._be._lib().j4q_decode_plan_run(self.handle, C.c_void_p(stream or None)), "decode plan run")

    def info(self) -> dict:
        d = N.DecodePlanDesc()
        check(self._be._lib().j4q_decode_plan_info(self.handle, C.byref(d)), "decode plan info")
        return {name: getattr(d, name) for name, _ in N.DecodePlanDesc._fields_}

    def destroy(self) -> None:
        check(self._be._lib().j4q_decode_plan_destroy(self.handle), "decode plan destroy")
        self.handle = 0


_DEFAULT: Mi355xBackend | None = None


def default_backend() -> Mi355xBackend:
    """BackendRegistry.defaultBackend for this engine (core/tensor/BackendRegistry.java:63-80).

    Honours the pin ``JAX4J_BACKEND`` (the Java system property ``jax4j.tensor.backend`` is
    mirrored by ``JAX4J_TENSOR_BACKEND``): a pinned name other than ``mi355x``, or a pinned
    ``mi355x`` without a usable gfx950 device, raises IllegalStateException.
    """
    global _DEFAULT
    pinned = os.environ.get("JAX4J_TENSOR_BACKEND") or os.environ.get("JAX4J_BACKEND")
    backend = _DEFAULT or Mi355xBackend()
    if pinned and pinned.strip():
        want = pinned.strip().lower()
        if want != backend.name() or not backend.is_available():
            raise IllegalStateException(f"Requested compute backend is unavailable: {want}")
    elif not backend.is_available():
        raise IllegalStateException("no nablatensor compute backend is available")
    _DEFAULT = backend
    return backend

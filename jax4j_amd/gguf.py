"""GGUF files for the quantized-matmul path: a host-side mirror of the engine's ``j4q_gguf_*``
entry points (include/jax4j_mi355x.h).

The reference takes quantized blobs from an external caller
(``QuantizedOps.uploadQuantized``, jax4j-core/.../tensor/spi/QuantizedOps.java:24) and
names the GGUF type ids in ``QuantType`` (jax4j-core/.../tensor/QuantType.java:3-13). A
``GGUFFile`` parses a .gguf file (v2/v3) in the engine library (memory-mapped, every length and
offset bounds-checked) and uploads a tensor's blocks straight into the engine.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _native as N
from .backend import Mi355xBackend, check
from .tensor import DeviceBuffer, Device, DType, QuantType

# GGUF metadata value types
GGUF_TYPES = {0: "u8", 1: "i8", 2: "u16", 3: "i16", 4: "u32", 5: "i32", 6: "f32", 7: "bool", 8: "string",
              9: "array", 10: "u64", 11: "i64", 12: "f64"}
_SCALAR_NP = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
              7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}


@dataclass(frozen=True)
class TensorInfo:
    index: int
    name: str
    type_id: int
    dims: tuple  # innermost first, as stored
    offset: int  # absolute file offset
    nbytes: int

    @property
    def shape(self) -> tuple:
        """Logical shape, outermost first: a matrix is (rows, cols)."""
        return tuple(reversed(self.dims))


class GGUFFile:
    """An open GGUF file (``j4q_gguf_open``); use as a context manager or call ``close()``."""

    def __init__(self, path: str):
        self._h = C.c_uint64()
        check(N.load().j4q_gguf_open(str(path).encode(), C.byref(self._h)), "gguf_open")
        info = N.GgufInfo()
        check(N.load().j4q_gguf_file_info(self._h, C.byref(info)), "gguf_file_info")
        self.version = info.version
        self.alignment = info.alignment
        self.data_offset = info.data_offset
        self.file_bytes = info.file_bytes
        self.tensors = [self._tensor(i) for i in range(info.tensor_count)]
        self.metadata = {}
        for i in range(info.metadata_count):
            key = C.create_string_buffer(1024)
            t, et, cnt = C.c_int32(), C.c_int32(), C.c_uint64()
            check(N.load().j4q_gguf_meta_key(self._h, i, key, 1024, C.byref(t), C.byref(et), C.byref(cnt)), "gguf_meta_key")
            self.metadata[key.value.decode()] = (GGUF_TYPES.get(t.value, str(t.value)), et.value, cnt.value)

    def _tensor(self, i: int) -> TensorInfo:
        t = N.GgufTensor()
        check(N.load().j4q_gguf_tensor_info(self._h, i, C.byref(t)), "gguf_tensor_info")
        return TensorInfo(i, t.name.decode(), t.type_id, tuple(t.dims[: t.n_dims]), t.offset, t.nbytes)

    def close(self) -> None:
        if self._h.value:
            check(N.load().j4q_gguf_close(self._h), "gguf_close")
            self._h = C.c_uint64()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def find(self, name: str) -> TensorInfo:
        idx = C.c_int64()
        check(N.load().j4q_gguf_find_tensor(self._h, name.encode(), C.byref(idx)), "gguf_find_tensor")
        return self.tensors[idx.value]

    def value(self, key: str):
        """Scalar or string metadata value (arrays: use ``metadata[key]`` for type and count)."""
        kind = self.metadata.get(key, ("", 0, 0))[0]
        if kind == "string":
            n = C.c_uint64()
            check(N.load().j4q_gguf_meta_string(self._h, key.encode(), None, 0, C.byref(n)), "gguf_meta_string")
            buf = C.create_string_buffer(n.value + 1)
            check(N.load().j4q_gguf_meta_string(self._h, key.encode(), buf, n.value + 1, None), "gguf_meta_string")
            return buf.raw[: n.value].decode()
        t = C.c_int32()
        raw = (C.c_uint8 * 8)()
        check(N.load().j4q_gguf_meta_scalar(self._h, key.encode(), C.byref(t), raw), "gguf_meta_scalar")
        dt = _SCALAR_NP[t.value]
        return np.frombuffer(bytes(raw)[: np.dtype(dt).itemsize], dtype=dt)[0].item()

    def read(self, tensor: TensorInfo | str) -> np.ndarray:
        """The tensor's raw blocks, copied to host memory."""
        t = self.find(tensor) if isinstance(tensor, str) else tensor
        out = np.empty(t.nbytes, np.uint8)
        check(N.load().j4q_gguf_read_tensor(self._h, t.index, out.ctypes.data_as(C.c_void_p), t.nbytes), "gguf_read_tensor")
        return out

    def upload(self, backend: Mi355xBackend, tensor: TensorInfo | str) -> DeviceBuffer:
        """uploadQuantized of the tensor straight from the mapped file."""
        t = self.find(tensor) if isinstance(tensor, str) else tensor
        lib = backend._lib()
        out = C.c_uint64()
        check(lib.j4q_gguf_upload(self._h, t.index, C.byref(out)), "gguf_upload")
        rows = int(np.prod(t.dims[1:], dtype=np.int64)) if len(t.dims) > 1 else 1
        return DeviceBuffer(out.value, (rows, t.dims[0]), DType.F32, Device.rocm(backend._device), QuantType.by_id(t.type_id))

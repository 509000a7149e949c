"""jax4j_amd: MI355X-native (gfx950) engine for jax4j's GGUF block-quantized matmul path.

The engine is the C-ABI library ``lib/libjax4j_mi355x.so`` (HIP kernels in ``csrc/``);
this package is its host-side mirror of the reference's QuantizedOps SPI.
"""
from .backend import Mi355xBackend, check, default_backend
from .tensor import (
    Device,
    DeviceBuffer,
    DeviceType,
    DType,
    IllegalArgumentException,
    IllegalStateException,
    QuantType,
    UnsupportedOperationException,
)

__all__ = [
    "Mi355xBackend",
    "default_backend",
    "check",
    "Device",
    "DeviceBuffer",
    "DeviceType",
    "DType",
    "IllegalArgumentException",
    "IllegalStateException",
    "QuantType",
    "UnsupportedOperationException",
]

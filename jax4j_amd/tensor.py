"""Host-side mirror of the reference's tensor SPI types for this path.

Names, argument meaning and error types follow jax4j 0.2.1 (paths relative to
``jax4j-core/src/main/java/com/nablatensor/jax4j/``):

- ``QuantType``            tensor/QuantType.java:4-53
- ``DType``                tensor/DType.java:19-35
- ``Device``/``DeviceType`` tensor/Device.java:19-55
- ``DeviceBuffer``         tensor/spi/DeviceBuffer.java:26-33
- Java exceptions map to ``IllegalArgumentException`` (a ``ValueError``),
  ``IllegalStateException`` and ``UnsupportedOperationException``.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field


class IllegalArgumentException(ValueError):
    """java.lang.IllegalArgumentException: bad type, shape, index or buffer."""


class IllegalStateException(RuntimeError):
    """java.lang.IllegalStateException: e.g. a pinned backend that is unavailable."""


class UnsupportedOperationException(NotImplementedError):
    """java.lang.UnsupportedOperationException: an op this backend does not provide."""


class QuantType(enum.Enum):
    """ggml block-quantization formats; ``id`` is the on-disk GGUF type id (QuantType.java:5-13)."""

    F32 = (0, 1, 4)
    F16 = (1, 1, 2)
    Q4_0 = (2, 32, 18)
    Q8_0 = (8, 32, 34)
    Q4_K = (12, 256, 144)
    Q6_K = (14, 256, 210)
    BF16 = (30, 1, 2)
    Q1_0 = (41, 256, 34)
    Q2_0 = (42, 128, 34)

    @property
    def id(self) -> int:
        return self.value[0]

    @property
    def block_elements(self) -> int:
        return self.value[1]

    @property
    def block_bytes(self) -> int:
        return self.value[2]

    @classmethod
    def by_id(cls, type_id: int) -> "QuantType":
        """QuantType.byId (QuantType.java:37-44)."""
        for t in cls:
            if t.id == type_id:
                return t
        raise IllegalArgumentException(f"unknown ggml quant type id: {type_id}")

    def byte_size_for(self, elements: int) -> int:
        """QuantType.byteSizeFor (QuantType.java:46-53)."""
        if elements % self.block_elements != 0:
            raise IllegalArgumentException(
                f"{self.name} tensor is not block-aligned: {elements} elements, block={self.block_elements}"
            )
        return (elements // self.block_elements) * self.block_bytes


class DType(enum.Enum):
    """tensor/DType.java:19-21 (the reference has no BF16; the engine adds it for GEMM inputs)."""

    F32 = "f32"
    F64 = "f64"
    F16 = "f16"
    I8 = "i8"
    I32 = "i32"
    I64 = "i64"
    BOOL = "bool"
    BF16 = "bf16"


class DeviceType(enum.Enum):
    CPU = "cpu"
    CUDA = "cuda"
    ROCM = "rocm"
    VULKAN = "vulkan"
    WGPU = "wgpu"


@dataclass(frozen=True)
class Device:
    """tensor/Device.java:19-55; the engine serves ``rocm:0``."""

    type: DeviceType = DeviceType.ROCM
    index: int = 0

    @staticmethod
    def rocm(index: int = 0) -> "Device":
        return Device(DeviceType.ROCM, index)

    def __str__(self) -> str:
        return f"{self.type.value}:{self.index}"


@dataclass
class DeviceBuffer:
    """An engine-owned buffer (spi/DeviceBuffer.java:26-33).

    For a quantized buffer ``shape`` is the logical F32 shape it decodes to and ``dtype`` is
    F32, as for the reference's CpuQuantBuffer (backend/cpu/CpuQuantBuffer.java:24-32);
    ``quant_type`` names the storage format.
    """

    handle: int
    shape: tuple
    dtype: DType
    device: Device = field(default_factory=Device.rocm)
    quant_type: QuantType | None = None

    def size(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

"""Writes GGUF files for the reader tests. A restatement of the published GGUF v3 layout
written independently of the C reader: header, metadata key/values, tensor infos, alignment
padding, tensor data."""
from __future__ import annotations

import struct

# GGUF metadata value types -> struct format of one scalar
SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
STRING, ARRAY = 8, 9


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype in SCALAR:
        return struct.pack(SCALAR[vtype], v)
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    raise ValueError(vtype)


def gguf_bytes(metadata, tensors, alignment=None, version=3) -> bytes:
    """metadata: [(key, vtype, value)]; tensors: [(name, type_id, dims innermost first, data)].
    Tensor data is placed in order, each at the next multiple of the alignment."""
    align = 32 if alignment is None else alignment
    md = list(metadata)
    if alignment is not None:
        md.append(("general.alignment", 4, alignment))
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(md))
    for key, vtype, v in md:
        out += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off = (off + len(data) + align - 1) // align * align
    for (name, tid, dims, _), o in zip(tensors, offsets):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", tid, o)
    out += b"\0" * ((-len(out)) % align)
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offsets):
        out += b"\0" * (base + o - len(out))
        out += bytes(data)
    return bytes(out)

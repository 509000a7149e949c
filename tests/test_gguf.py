"""GGUF reader (the engine's j4q_gguf_* entry points) on the CPU: header, metadata, tensor
infos, alignment, type ids and byte-exact tensor data, plus the malformed-file errors. The
files are written by tests/gguf_fixtures.py, an independent restatement of the format."""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

from jax4j_amd import IllegalArgumentException, QuantType
from jax4j_amd import _native as N
from jax4j_amd import synthetic as S
from jax4j_amd.gguf import GGUFFile

from gguf_fixtures import ARRAY, STRING, gguf_bytes

MATS = [("blk.0.attn_q.weight", QuantType.Q4_0, 48, 256), ("blk.0.ffn_down.weight", QuantType.Q6_K, 20, 512),
        ("blk.0.ffn_up.weight", QuantType.Q4_K, 40, 256), ("output.weight", QuantType.Q8_0, 33, 96)]
META = [("general.architecture", STRING, "llama"), ("llama.context_length", 4, 8192), ("general.file_type", 4, 15),
        ("test.i8", 1, -7), ("test.u16", 2, 65535), ("test.i64", 11, -(1 << 40)), ("test.f32", 6, 1.5),
        ("test.f64", 12, -2.25), ("test.bool", 7, True), ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<s>", "</s>", "a"])),
        ("test.nested", ARRAY, (ARRAY, [(4, [1, 2]), (4, [3])]))]


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def model_file(tmp_path, alignment=None):
    tensors = [(n, qt.id, [cols, rows], S.quant_blocks(qt, 7 + rows, rows, cols).tobytes()) for n, qt, rows, cols in MATS]
    norm = np.linspace(-1, 1, 256).astype(np.float32)
    tensors.append(("blk.0.attn_norm.weight", 0, [256], norm.tobytes()))
    return write(tmp_path, "model.gguf", gguf_bytes(META, tensors, alignment)), tensors


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_gguf_tensors_and_data(tmp_path, alignment):
    path, tensors = model_file(tmp_path, alignment)
    raw = path.read_bytes()
    with GGUFFile(path) as f:
        assert f.version == 3 and f.alignment == (alignment or 32)
        assert f.data_offset % f.alignment == 0 and f.file_bytes == len(raw)
        assert [t.name for t in f.tensors] == [t[0] for t in tensors]
        for (name, tid, dims, data), t in zip(tensors, f.tensors):
            assert (t.type_id, list(t.dims), t.nbytes) == (tid, dims, len(data))
            assert t.offset % f.alignment == 0
            assert raw[t.offset:t.offset + t.nbytes] == data
            assert f.read(t).tobytes() == data
        q = f.find("blk.0.attn_q.weight")
        assert q.shape == (48, 256) and q.type_id == QuantType.Q4_0.id
        # QuantType.byteSizeFor (QuantType.java:46-53) agrees with the reader's sizes
        for name, qt, rows, cols in MATS:
            assert f.find(name).nbytes == qt.byte_size_for(rows * cols)


def test_gguf_metadata(tmp_path):
    path, _ = model_file(tmp_path)
    with GGUFFile(path) as f:
        assert f.value("general.architecture") == "llama"
        assert f.value("llama.context_length") == 8192
        assert f.value("test.i8") == -7 and f.value("test.u16") == 65535
        assert f.value("test.i64") == -(1 << 40)
        assert f.value("test.f32") == 1.5 and f.value("test.f64") == -2.25 and f.value("test.bool") is True
        assert f.metadata["tokenizer.ggml.tokens"] == ("array", STRING, 3)
        assert f.metadata["test.nested"] == ("array", ARRAY, 2)
        with pytest.raises(IllegalArgumentException, match="not a scalar"):
            f.value("tokenizer.ggml.tokens")
        with pytest.raises(IllegalArgumentException, match="no metadata key"):
            f.value("missing.key")
        with pytest.raises(IllegalArgumentException, match="no tensor named"):
            f.find("missing.weight")


def test_gguf_version2_and_empty(tmp_path):
    p = write(tmp_path, "v2.gguf", gguf_bytes([("a", 4, 1)], [], version=2))
    with GGUFFile(p) as f:
        assert f.version == 2 and f.tensors == [] and f.value("a") == 1


def corrupt(data: bytes, pos: int, new: bytes) -> bytes:
    return data[:pos] + new + data[pos + len(new):]


def test_gguf_rejects_malformed_files(tmp_path):
    path, _ = model_file(tmp_path)
    good = path.read_bytes()
    cases = {
        "bad magic": corrupt(good, 0, b"GGUX"),
        "truncated header": good[:10],
        "truncated metadata": good[:200],
        "huge tensor count": corrupt(good, 8, struct.pack("<Q", 1 << 60)),
        "huge string": corrupt(good, 24, struct.pack("<Q", 1 << 40)),
        "data past the end": good[: len(good) - 100],
    }
    for what, data in cases.items():
        p = write(tmp_path, "bad.gguf", data)
        with pytest.raises(IllegalArgumentException, match="GGUF"):
            GGUFFile(p)
    p = write(tmp_path, "v9.gguf", corrupt(good, 4, struct.pack("<I", 9)))
    with pytest.raises(Exception, match="version 9"):
        GGUFFile(p)
    # a tensor offset that is not a multiple of the alignment
    tensors = [("t", QuantType.Q8_0.id, [32, 1], bytes(34))]
    data = bytearray(gguf_bytes([], tensors))
    name_end = 4 + 4 + 8 + 8 + 8 + 1 + 4 + 16 + 4
    data[name_end:name_end + 8] = struct.pack("<Q", 3)
    p = write(tmp_path, "misaligned.gguf", bytes(data))
    with pytest.raises(IllegalArgumentException, match="alignment"):
        GGUFFile(p)
    # a row that is not a whole number of blocks
    p = write(tmp_path, "ragged.gguf", gguf_bytes([], [("t", QuantType.Q4_K.id, [100, 2], bytes(144))]))
    with pytest.raises(IllegalArgumentException, match="multiple of its block"):
        GGUFFile(p)
    with pytest.raises(IllegalArgumentException, match="cannot open"):
        GGUFFile(tmp_path / "missing.gguf")


def test_gguf_handles(tmp_path):
    path, _ = model_file(tmp_path)
    lib = N.load()
    h = C.c_uint64()
    assert lib.j4q_gguf_open(str(path).encode(), C.byref(h)) == N.J4Q_OK
    assert lib.j4q_gguf_close(h) == N.J4Q_OK
    info = N.GgufInfo()
    assert lib.j4q_gguf_file_info(h, C.byref(info)) == N.J4Q_EHANDLE
    assert lib.j4q_gguf_close(0) == N.J4Q_OK
    t = N.GgufTensor()
    assert lib.j4q_gguf_tensor_info(0, 0, C.byref(t)) == N.J4Q_EHANDLE

"""GGUF tensors uploaded straight from the mapped file (j4q_gguf_upload) on the GPU: the
layout round trip is bit-exact and the GEMV matches the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from jax4j_amd import IllegalArgumentException, QuantType
from jax4j_amd import synthetic as S
from jax4j_amd.gguf import GGUFFile

from gguf_fixtures import gguf_bytes

pytestmark = pytest.mark.gpu

MATS = [("q", QuantType.Q4_0, 48, 256), ("down", QuantType.Q6_K, 20, 512), ("up", QuantType.Q4_K, 40, 256),
        ("out", QuantType.Q8_0, 33, 96), ("pilot", QuantType.Q2_0, 9, 256)]


def test_gguf_upload_round_trip_and_gemv(backend, tmp_path):
    print("[case] gguf upload", flush=True)
    blobs = {n: S.quant_blocks(qt, 11 + rows, rows, cols) for n, qt, rows, cols in MATS}
    tensors = [(n, qt.id, [cols, rows], blobs[n].tobytes()) for n, qt, rows, cols in MATS]
    tensors.append(("norm", 0, [64], np.ones(64, np.float32).tobytes()))
    path = tmp_path / "m.gguf"
    path.write_bytes(gguf_bytes([("general.architecture", 8, "llama")], tensors, alignment=64))
    with GGUFFile(path) as f:
        for n, qt, rows, cols in MATS:
            w = f.upload(backend, n)
            assert w.shape == (rows, cols) and w.quant_type == qt
            assert np.array_equal(backend.export_quantized(w), blobs[n])
            x = S.activations_f32(5 + rows, cols)
            xb = backend.upload(x)
            y = backend.quant_matvec(w, xb)
            ref = oracle.matvec_f64(qt.id, blobs[n], rows, cols, x)
            got = backend.download(y).astype(np.float64)
            assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
            for h in (w, xb, y):
                backend.release(h)
        # an F32 tensor is not a quantized type uploadQuantized accepts
        with pytest.raises(IllegalArgumentException):
            f.upload(backend, "norm")

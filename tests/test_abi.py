"""The C-ABI library on a machine without a GPU: loading, exported symbols, the quant-type
table, host-side argument checks and the host generator. No kernel is launched here."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from jax4j_amd import _native as N
from jax4j_amd import IllegalArgumentException, IllegalStateException, QuantType
from jax4j_amd import backend as B
from jax4j_amd import synthetic as S

HEADER = Path(__file__).resolve().parents[1] / "include" / "jax4j_mi355x.h"


def header_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^(?:int|const char \*)\s*(j4q_\w+)\(", text, flags=re.M))


def test_library_exports_every_declared_symbol():
    lib = N.load()
    declared = header_functions()
    assert len(declared) >= 30
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert declared == set(N.SIGNATURES), "ctypes binding and header disagree"
    assert lib.j4q_abi_version() == 1


def test_probe_never_raises():
    assert N.load().j4q_probe() in (0, 1)
    assert isinstance(B.Mi355xBackend().is_available(), bool)


def test_quant_type_table_matches_reference_enum():
    # core/tensor/QuantType.java:5-13
    expected = {"Q4_0": (2, 32, 18), "Q8_0": (8, 32, 34), "Q4_K": (12, 256, 144), "Q6_K": (14, 256, 210), "Q2_0": (42, 128, 34)}
    lib = N.load()
    for name, (tid, be, bb) in expected.items():
        qt = QuantType[name]
        assert (qt.id, qt.block_elements, qt.block_bytes) == (tid, be, bb)
        e, b = C.c_int32(), C.c_int32()
        assert lib.j4q_quant_type_info(tid, C.byref(e), C.byref(b)) == N.J4Q_OK
        assert (e.value, b.value) == (be, bb)
        out = C.c_uint64()
        assert lib.j4q_quant_byte_size(tid, 4096 * 4096, C.byref(out)) == N.J4Q_OK
        assert out.value == qt.byte_size_for(4096 * 4096) == 4096 * 4096 // be * bb
        assert lib.j4q_quant_byte_size(tid, be + 1, C.byref(out)) == N.J4Q_EINVAL
    assert lib.j4q_quant_type_info(0, None, None) == N.J4Q_EUNSUPPORTED  # F32 is not block-quantized
    with pytest.raises(IllegalArgumentException, match="not block-aligned"):
        QuantType.Q4_K.byte_size_for(300)
    with pytest.raises(IllegalArgumentException, match="unknown ggml quant type id"):
        QuantType.by_id(3)


def test_supported_quant_types():
    be = B.Mi355xBackend()
    assert be.supported_quant_types() == {QuantType.Q2_0, QuantType.Q4_0, QuantType.Q8_0, QuantType.Q4_K, QuantType.Q6_K}


@pytest.mark.parametrize(
    "qt_id,nbytes,rows,cols,code",
    [
        (3, 18, 1, 32, N.J4Q_EINVAL),  # no such GGUF id
        (30, 2, 1, 1, N.J4Q_EUNSUPPORTED),  # BF16 exists but is not a block format here
        (2, 18, 1, 33, N.J4Q_EINVAL),  # cols not block-aligned
        (2, 18, 0, 32, N.J4Q_EINVAL),  # rows <= 0
        (2, 17, 1, 32, N.J4Q_EINVAL),  # wrong byte count
        (12, 144, 1, 128, N.J4Q_EINVAL),  # Q4_K needs cols % 256 == 0
        (14, 210 * 2, 2, 256, N.J4Q_OK),  # valid: fails later only for want of a device
    ],
)
def test_upload_quantized_argument_checks_before_any_hip_call(qt_id, nbytes, rows, cols, code):
    lib = N.load()
    blob = np.zeros(max(nbytes, 1), dtype=np.uint8)
    out = C.c_uint64()
    rc = lib.j4q_upload_quantized(qt_id, blob.ctypes.data_as(C.c_void_p), nbytes, rows, cols, C.byref(out))
    if code == N.J4Q_OK:
        assert rc in (N.J4Q_OK, N.J4Q_ENODEV)
        if rc == N.J4Q_OK:
            assert lib.j4q_release(out.value) == N.J4Q_OK
    else:
        assert rc == code
        assert N.last_error()


def test_stale_and_foreign_handles_rejected():
    lib = N.load()
    out = C.c_uint64()
    assert lib.j4q_quant_matvec(0xDEAD00000001, 0x1, C.byref(out)) == N.J4Q_EHANDLE
    assert "handle" in N.last_error()
    assert lib.j4q_release(0) == N.J4Q_OK
    assert lib.j4q_release(12345) == N.J4Q_EHANDLE


def test_raw_entry_points_check_alignment_and_batch():
    lib = N.load()
    rc = lib.j4q_quant_matvec_into(1, C.c_void_p(0x1001), None, C.c_void_p(0x2000), 1, None)
    assert rc == N.J4Q_EINVAL and "aligned" in N.last_error()
    rc = lib.j4q_quant_matvec_into(1, C.c_void_p(0x1000), None, C.c_void_p(0x2000), 0, None)
    assert rc == N.J4Q_EINVAL


def test_gemv_policy_round_trip_and_unknown_policy():
    lib = N.load()
    prev = C.c_int(-1)
    assert lib.j4q_set_gemv_policy(7, C.byref(prev)) == N.J4Q_EINVAL and "policy" in N.last_error()
    assert prev.value == -1  # nothing changed, nothing written
    assert lib.j4q_set_gemv_policy(N.GEMV_FP32, C.byref(prev)) == N.J4Q_OK
    assert prev.value == N.GEMV_MATRIX_CORES
    assert lib.j4q_set_gemv_policy(N.GEMV_MATRIX_CORES, None) == N.J4Q_OK
    assert lib.j4q_set_gemv_policy(N.GEMV_MATRIX_CORES, C.byref(prev)) == N.J4Q_OK
    assert prev.value == N.GEMV_MATRIX_CORES
    be = B.Mi355xBackend.__new__(B.Mi355xBackend)  # the setter needs no device
    with pytest.raises(IllegalArgumentException):
        be.set_gemv_policy("bf16")
    assert be.set_gemv_policy("fp32") == "matrix_cores"
    assert be.set_gemv_policy("matrix_cores") == "fp32"


def test_error_mapping_follows_reference_exception_types():
    with pytest.raises(IllegalArgumentException):
        B.check(N.J4Q_EINVAL, "x")
    with pytest.raises(IllegalArgumentException):
        B.check(N.J4Q_EHANDLE, "x")
    with pytest.raises(IllegalStateException):
        B.check(N.J4Q_ENODEV, "x")
    with pytest.raises(RuntimeError):
        B.check(N.J4Q_EHIP, "x")


def test_backend_pin_by_name(monkeypatch):
    # BackendRegistry.defaultBackend (core/tensor/BackendRegistry.java:63-72)
    monkeypatch.setenv("JAX4J_BACKEND", "cuda")
    with pytest.raises(IllegalStateException, match="unavailable: cuda"):
        B.default_backend()
    monkeypatch.setenv("JAX4J_BACKEND", "mi355x")
    if not B.Mi355xBackend().is_available():
        with pytest.raises(IllegalStateException, match="unavailable: mi355x"):
            B.default_backend()


def test_host_generator_deterministic_and_distributed():
    a = S.quant_blocks(QuantType.Q4_K, 5, 8, 512)
    b = S.quant_blocks(QuantType.Q4_K, 5, 8, 512)
    c = S.quant_blocks(QuantType.Q4_K, 6, 8, 512)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    x = S.activations_f32(1, 200_000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    q8 = S.quant_blocks(QuantType.Q8_0, 9, 64, 4096).reshape(-1, 34)
    q = q8[:, 2:].view(np.int8)
    assert q.min() == -127 and q.max() == 127
    d = q8[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and abs(d.mean() / 0.02 - np.sqrt(2 / np.pi)) < 0.02  # E|N(0,1)| = sqrt(2/pi)

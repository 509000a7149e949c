"""j4q_quant_matmul_noalloc: the prefill GEMM whose int8 workspace is the engine's fixed device
array instead of an allocation, against j4q_quant_matmul_into with a caller workspace,
through the C ABI.

Bar: bit for bit (the same kernels run on the same operands), for both variants, on two
calls in a row where the second is smaller (the workspace keeps the first call's contents),
and at the workspace's limit; a call above the limit is refused before anything runs.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

from jax4j_amd import DType, QuantType
from jax4j_amd import _native as N
from jax4j_amd import synthetic as S

pytestmark = pytest.mark.gpu

LIMIT = 32 << 20  # m * cols of the int8 workspace


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def ptr(backend, buf):
    return backend.buffer_desc(buf).device_ptr


def reference(backend, w, xp, m, k, n, variant, yp):
    """j4q_quant_matmul_into with the caller's own workspace."""
    xq = backend.upload(np.zeros((m * k + 3) // 4, np.float32))
    xs = backend.upload(np.zeros(m * (k // 32), np.float32))
    rc = N.load().j4q_quant_matmul_into(w.handle, C.c_void_p(xp), m, variant, C.c_void_p(ptr(backend, xq)),
                                        C.c_void_p(ptr(backend, xs)), C.c_void_p(yp), None)
    assert rc == 0, N.last_error()
    backend.sync()
    backend.release(xq)
    backend.release(xs)


@pytest.mark.parametrize("variant", [N.GEMM_INT8, N.GEMM_BF16], ids=["int8", "bf16"])
def test_noalloc_matches_into_twice_and_at_the_limit(backend, variant):
    lib = N.load()
    cases = [(512, 1024, 4096), (37, 1024, 4096), (8192, 256, 4096)]  # second smaller; third m * k = limit
    for m, n, k in cases:
        note("noalloc", "int8" if variant == N.GEMM_INT8 else "bf16", m, n, k)
        assert m * k <= LIMIT
        wblob = S.quant_blocks(QuantType.Q8_0, 0x5EED8 + m, n, k)
        w = backend.upload_quantized(wblob, QuantType.Q8_0, (n, k))
        x = backend.upload(S.activations_bf16(m + 1, m * k), shape=(m, k), dtype=DType.BF16)
        y_ref = backend.upload(np.zeros(m * n, np.float32))
        y = backend.upload(np.full(m * n, np.nan, np.float32))
        reference(backend, w, ptr(backend, x), m, k, n, variant, ptr(backend, y_ref))
        rc = lib.j4q_quant_matmul_noalloc(w.handle, C.c_void_p(ptr(backend, x)), m, variant,
                                          C.c_void_p(ptr(backend, y)), None)
        assert rc == 0, N.last_error()
        backend.sync()
        got, want = backend.download(y), backend.download(y_ref)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"m={m}"
        for b in (w, x, y_ref, y):
            backend.release(b)


def test_noalloc_refuses_above_the_workspace(backend):
    lib = N.load()
    m, n, k = LIMIT // 4096 + 1, 64, 4096
    w = backend.upload_quantized(S.quant_blocks(QuantType.Q8_0, 3, n, k), QuantType.Q8_0, (n, k))
    x = backend.upload(np.zeros(m * k, np.uint16), shape=(m, k), dtype=DType.BF16)
    y = backend.upload(np.zeros(m * n, np.float32))
    rc = lib.j4q_quant_matmul_noalloc(w.handle, C.c_void_p(ptr(backend, x)), m, N.GEMM_INT8, C.c_void_p(ptr(backend, y)), None)
    assert rc == N.J4Q_EUNSUPPORTED and "workspace" in N.last_error()
    for b in (w, x, y):
        backend.release(b)

"""j4q_gemv_trace: the per-wave timeline of a batch-1 GEMV launch (engine-local measurement).

One launch of the vector-ALU GEMV with the trace set writes, for every wave of the grid, its
entry time, the time its x image was staged, the time its last item was done and its item
count; the GEMV's result is the same with and without the trace.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import oracle
from jax4j_amd import IllegalArgumentException, QuantType
from jax4j_amd import _native as N
from jax4j_amd import synthetic as S
from jax4j_amd.backend import check

pytestmark = pytest.mark.gpu


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("qt,rows,cols", [(QuantType.Q4_K, 3000, 4096), (QuantType.Q6_K, 1000, 14336)])
def test_gemv_trace_records_every_wave(backend, qt, rows, cols):
    note("gemv trace", qt.name, rows, cols)
    lib = N.load()
    blob = S.quant_blocks(qt, 0x7A, rows, cols)
    x = S.activations_f32(0x7B, cols)
    w = backend.upload_quantized(blob, qt, (rows, cols))
    xb = backend.upload(x)
    y0 = backend.quant_matvec(w, xb)
    ref = backend.download(y0)
    words = 4 * 65536
    buf = backend.upload(np.zeros(words * 2, np.float32))  # words x 8 bytes of zeros
    bp = backend.buffer_desc(buf).device_ptr
    with pytest.raises(IllegalArgumentException, match="4 words"):
        check(lib.j4q_gemv_trace(C.c_void_p(bp), 3), "gemv_trace")
    assert lib.j4q_gemv_trace(C.c_void_p(bp), words) == 0
    try:
        y = backend.quant_matvec(w, xb)
    finally:
        assert lib.j4q_gemv_trace(None, 0) == 0
    got = backend.download(y)
    # the trace does not change the result
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.abs(got.astype(np.float64) - oracle.matvec_f64(qt.id, blob, rows, cols, x)).max() <= 1e-5 * np.abs(ref).max()
    t = backend.download_raw(buf).view(np.uint64).reshape(-1, 4)
    live = t[t[:, 0] != 0]
    nw = len(live)
    assert nw > 0 and nw % 8 == 0  # whole workgroups of 8 or 16 waves
    assert np.all(live[:, 0] <= live[:, 1]) and np.all(live[:, 1] <= live[:, 2])
    items = (live[:, 3] & 0xFFFFFFFF).astype(np.int64)
    cpl = (cols // 32 + 63) // 64
    # rows go to waves round-robin: every row's chunk steps are somebody's items, once
    assert items.sum() == rows * cpl
    assert items.max() - items.min() <= cpl
    for h in (w, xb, y0, y, buf):
        backend.release(h)

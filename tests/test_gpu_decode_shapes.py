"""configs[4] (Llama-3-8B-shaped decode step, Q4_K_M mix) at its real matrix shapes, against the
CPU oracle, through the C ABI.

Every GEMV the decode step launches is checked here at full size and at the batch sizes the
benchmark runs (1 and 16): the 128256 x 4096 Q6_K output head, the per-layer Q4_K and Q6_K
matrices, and the row concatenations (q|k|v 6144 x 4096, gate|up 28672 x 4096) the step runs
as single launches. The semantics are quantMatvec / quantMatvecAdd per batch row
(QuantizedOps.java:27-30; CpuBackend.java:708-736).

Bars: the vector-ALU kernel (B = 1) within 1e-5 * ||y_ref||_inf of the fp64 oracle, the
matrix-core kernel (B = 16) within 4e-5 (its block sums round one way, so the error grows
with K; measured 1.0e-5 at K = 11008), both far inside the decode tolerance of 1e-3. A
quantMatvecAdd result is fl(W.x) + add bit for bit.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import oracle
from jax4j_amd import DType, IllegalArgumentException, QuantType, check
from jax4j_amd import _native as N
from jax4j_amd import synthetic as S

pytestmark = pytest.mark.gpu

Q4K, Q6K = QuantType.Q4_K, QuantType.Q6_K
TOL_B1, TOL_B16 = 1e-5, 4e-5


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def rel_err(y, y_ref):
    return float(np.abs(y.astype(np.float64) - y_ref).max() / max(np.abs(y_ref).max(), 1e-30))


def device_matrix(backend, qt, rows, cols, seed):
    """GGUF blocks generated on the device (bit-identical to the host generator, checked in
    test_gpu_parity), copied back for the oracle and uploaded from device memory."""
    nbytes = qt.byte_size_for(rows * cols)
    raw = backend.upload(np.zeros((nbytes + 3) // 4, np.float32))
    ptr = backend.buffer_desc(raw).device_ptr
    check(N.load().j4q_synth_quant_device(qt.id, seed, rows, cols, C.c_void_p(ptr), nbytes, None), "synth")
    backend.sync()
    blob = backend.download(raw).view(np.uint8)[:nbytes].copy()
    w = backend.upload_quantized_device(ptr, nbytes, qt, (rows, cols))
    backend.release(raw)
    return blob, w


def run(backend, w, xs, add=None):
    B, cols = xs.shape
    rows = w.shape[0]
    xb = backend.upload(xs if B > 1 else xs[0], shape=(B, cols) if B > 1 else None)
    if add is None:
        y = backend.quant_matvec(w, xb)
    else:
        ab = backend.upload(add if B > 1 else add[0], shape=(B, rows) if B > 1 else None)
        y = backend.quant_matvec_add(w, xb, ab)
        backend.release(ab)
    got = backend.download(y).reshape(B, rows)
    backend.release(y)
    backend.release(xb)
    return got


def test_output_head_128256x4096_q6k_b1_b16(backend):
    rows, cols = 128256, 4096
    note("head", rows, cols)
    blob, w = device_matrix(backend, Q6K, rows, cols, 0xDEC0DE + 224)
    xs = S.activations_f32(0xA11, 16 * cols).reshape(16, cols)
    ref = oracle.matmul_f64(Q6K.id, blob, rows, cols, xs)
    g1 = run(backend, w, xs[:1])
    assert rel_err(g1[0], ref[0]) <= TOL_B1
    g16 = run(backend, w, xs)
    for b in range(16):
        assert rel_err(g16[b], ref[b]) <= TOL_B16, f"batch row {b}"
    add = S.activations_f32(0xA13, 16 * rows).reshape(16, rows)
    ga = run(backend, w, xs, add)
    assert np.array_equal(bits(ga), bits(g16 + add))
    backend.release(w)


LAYER = [
    ("q/o", Q4K, 4096, 4096),
    ("k/v", Q4K, 1024, 4096),
    ("gate/up", Q4K, 14336, 4096),
    ("down", Q6K, 4096, 14336),
]


@pytest.mark.parametrize("name,qt,rows,cols", LAYER, ids=[l[0] for l in LAYER])
def test_layer_matrix_b1_b16(backend, name, qt, rows, cols):
    note("layer", name, qt.name, rows, cols)
    blob, w = device_matrix(backend, qt, rows, cols, 0xDEC0DE + rows + cols)
    xs = S.activations_f32(cols + 1, 16 * cols).reshape(16, cols)
    ref = oracle.matmul_f64(qt.id, blob, rows, cols, xs)
    g1 = run(backend, w, xs[:1])
    assert rel_err(g1[0], ref[0]) <= TOL_B1
    g16 = run(backend, w, xs)
    for b in range(16):
        assert rel_err(g16[b], ref[b]) <= TOL_B16, f"batch row {b}"
    backend.release(w)


FUSED = [("qkv", Q4K, [4096, 1024, 1024], 4096), ("gate|up", Q4K, [14336, 14336], 4096)]


@pytest.mark.parametrize("name,qt,parts,cols", FUSED, ids=[f[0] for f in FUSED])
@pytest.mark.parametrize("B", [1, 16])
def test_fused_concat_matrices(backend, name, qt, parts, cols, B):
    """The row concatenations the decode step runs as one launch: the fused output is each
    part's output bit for bit, and matches the oracle on the concatenated blocks."""
    note("fused", name, parts, cols, "B", B)
    made = [device_matrix(backend, qt, r, cols, 0xF00 + 7 * i + r) for i, r in enumerate(parts)]
    fused = backend.concat_rows([w for _, w in made])
    rows = sum(parts)
    assert fused.shape == (rows, cols)
    xs = S.activations_f32(rows + B, B * cols).reshape(B, cols)
    got = run(backend, fused, xs)
    off = 0
    for (_, w), r in zip(made, parts):
        assert np.array_equal(bits(got[:, off:off + r]), bits(run(backend, w, xs))), f"part at row {off}"
        off += r
    ref = oracle.matmul_f64(qt.id, np.concatenate([b for b, _ in made]), rows, cols, xs)
    for b in range(B):
        assert rel_err(got[b], ref[b]) <= (TOL_B1 if B == 1 else TOL_B16), f"batch row {b}"
    for _, w in made:
        backend.release(w)
    backend.release(fused)


@pytest.mark.parametrize("name,qt,rows,cols", [LAYER[0], LAYER[3]], ids=["o", "down"])
@pytest.mark.parametrize("B", [1, 16])
def test_residual_add_in_place_full_size(backend, name, qt, rows, cols, B):
    """The residual update of a decoder layer: h = W.x + h with y on the add buffer itself
    (quantMatvecAdd in place through the stream-ordered entry point)."""
    note("residual in place", name, qt.name, rows, cols, "B", B)
    blob, w = device_matrix(backend, qt, rows, cols, 0xBEEF + rows + cols)
    xs = S.activations_f32(cols + 3, B * cols).reshape(B, cols)
    h0 = S.activations_f32(rows + 4, B * rows).reshape(B, rows)
    xb = backend.upload(xs if B > 1 else xs[0], shape=(B, cols) if B > 1 else None)
    hb = backend.upload(h0 if B > 1 else h0[0], shape=(B, rows) if B > 1 else None)
    hp = backend.buffer_desc(hb).device_ptr
    backend.quant_matvec_into(w, backend.buffer_desc(xb).device_ptr, hp, hp, B)
    backend.sync()
    got = backend.download(hb).reshape(B, rows)
    ref = oracle.matmul_f64(qt.id, blob, rows, cols, xs) + h0.astype(np.float64)
    for b in range(B):
        assert rel_err(got[b], ref[b]) <= (TOL_B1 if B == 1 else TOL_B16), f"batch row {b}"
    if B == 1:  # the same single-pass kernel as the out-of-place call: fl(W.x) + h bit for bit
        y = run(backend, w, xs)
        assert np.array_equal(bits(got), bits(y + h0))
    for h in (xb, hb, w):
        backend.release(h)


def test_rejected_calls_leave_no_live_buffer(backend):
    """A call refused for its size allocates nothing; the engine's live-buffer count and bytes
    are the same before and after."""
    qt, cols = QuantType.Q8_0, 32
    w = backend.upload_quantized(S.quant_blocks(qt, 9, 32, cols), qt, (32, cols))
    m = 65535 * 64 + 1  # above the prefill GEMM's row limit
    x = backend.upload(np.zeros(m * cols, np.uint16), shape=(m, cols), dtype=DType.BF16)
    before = backend.buffer_stats()
    for variant in ("int8", "bf16"):
        with pytest.raises(IllegalArgumentException, match="GEMM limits"):
            backend.quant_matmul(w, x, variant)
    assert backend.buffer_stats() == before
    backend.release(x)
    backend.release(w)

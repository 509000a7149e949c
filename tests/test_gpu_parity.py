"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars: dequantized weights and layout round trips are bit-exact; GEMV outputs are within
max|dy| <= 1e-3 * ||y_ref||_inf of the fp64 oracle (and one-hot / known-answer cases are
exact, since every partial sum there is exactly representable).
"""
from __future__ import annotations

import json
import sys
import threading
from pathlib import Path

import numpy as np
import pytest

import oracle
from jax4j_amd import IllegalArgumentException, QuantType
from jax4j_amd import synthetic as S

pytestmark = pytest.mark.gpu

KAT = json.loads((Path(__file__).parent / "golden" / "kat_blocks.json").read_text())["cases"]
FORMATS = [QuantType.Q4_0, QuantType.Q8_0, QuantType.Q4_K, QuantType.Q6_K, QuantType.Q2_0]
TOL = 1e-3

# (rows, cols) per format: small/odd shapes plus the benchmark shapes.
SHAPES = {
    QuantType.Q4_0: [(1, 32), (13, 96), (257, 2080), (11008, 4096)],
    QuantType.Q8_0: [(1, 32), (13, 96), (257, 2080), (4096, 4096)],
    QuantType.Q4_K: [(1, 256), (13, 768), (257, 2304), (1024, 4096), (14336, 4096)],
    QuantType.Q6_K: [(1, 256), (13, 768), (257, 2304), (4096, 14336)],
    QuantType.Q2_0: [(1, 128), (13, 384), (257, 2176), (4096, 4096)],
}
CASES = [(qt, r, c) for qt in FORMATS for (r, c) in SHAPES[qt]]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def rel_err(y, y_ref):
    return float(np.abs(y.astype(np.float64) - y_ref).max() / max(np.abs(y_ref).max(), 1e-30))


@pytest.fixture(scope="module")
def uploaded(backend):
    """One uploaded matrix per case, shared by the tests of this module."""
    cache = {}

    def get(qt, rows, cols, seed=0x5EED5):
        key = (qt, rows, cols, seed)
        if key not in cache:
            blob = S.quant_blocks(qt, seed + rows + cols, rows, cols)
            cache[key] = (blob, backend.upload_quantized(blob, qt, (rows, cols)))
        return cache[key]

    yield get
    for _, w in cache.values():
        backend.release(w)


@pytest.mark.parametrize("qt,rows,cols", CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_export_round_trip_bit_exact(backend, uploaded, qt, rows, cols):
    note("export", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    assert np.array_equal(backend.export_quantized(w), blob)


@pytest.mark.parametrize("qt,rows,cols", CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_gather_row_bit_exact(backend, uploaded, qt, rows, cols):
    note("gather", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    for r in sorted({0, rows // 2, rows - 1}):
        y = backend.quant_gather_row(w, r)
        got = backend.download(y)
        backend.release(y)
        assert np.array_equal(bits(got), bits(oracle.gather_row(qt.id, blob, r, rows, cols))), f"row {r}"


@pytest.mark.parametrize("qt,rows,cols", [c for c in CASES if c[1] * c[2] <= 1 << 22], ids=lambda v: getattr(v, "name", str(v)))
def test_dequantize_matrix_bit_exact(backend, uploaded, qt, rows, cols):
    note("dequantize", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    y = backend.dequantize(w)
    got = backend.download(y).reshape(rows, cols)
    backend.release(y)
    assert np.array_equal(bits(got), bits(oracle.dequant_matrix(qt.id, blob, rows, cols)))


@pytest.mark.parametrize("case", KAT, ids=[c["name"] for c in KAT])
def test_gemv_known_answers_exact(backend, case):
    note("kat", case["name"])
    qt = QuantType.by_id(case["type_id"])
    blob = np.frombuffer(bytes.fromhex(case["blob_hex"]), dtype=np.uint8)
    k = case["cols"]
    w = backend.upload_quantized(blob, qt, (1, k))
    for x, want in ((np.ones(k, np.float32), case["gemv_x_ones"]), (((np.arange(k) % 7) - 3).astype(np.float32), case["gemv_x_ramp"])):
        xb = backend.upload(x)
        y = backend.quant_matvec(w, xb)
        assert backend.download(y)[0] == np.float32(want)
        backend.release(y)
        backend.release(xb)
    g = backend.quant_gather_row(w, 0)
    assert np.array_equal(bits(backend.download(g)), bits(np.array(case["values"], np.float32)))
    backend.release(g)
    backend.release(w)


@pytest.mark.parametrize("qt", FORMATS, ids=lambda q: q.name)
def test_gemv_one_hot_returns_column_exactly(backend, uploaded, qt):
    rows, cols = SHAPES[qt][2]
    note("onehot", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    wd = oracle.dequant_matrix(qt.id, blob, rows, cols)
    for j in (0, 31, cols // 2 + 3, cols - 1):
        x = np.zeros(cols, np.float32)
        x[j] = 1.0
        xb = backend.upload(x)
        y = backend.quant_matvec(w, xb)
        got = backend.download(y)
        # the column itself (values; a -0.0 weight sums to +0.0 from the +0.0 start) and,
        # bit for bit, the reference loop's result (float sum = 0.0f; CpuQ4Gemm.java:30)
        assert np.array_equal(got, wd[:, j]), f"column {j}"
        assert np.array_equal(bits(got), bits(oracle.matvec(qt.id, blob, rows, cols, x))), f"column {j}"
        backend.release(y)
        backend.release(xb)


@pytest.mark.parametrize("qt,rows,cols", CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_gemv_matches_oracle(backend, uploaded, qt, rows, cols):
    note("gemv", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    x = S.activations_f32(rows * 31 + cols, cols)
    xb = backend.upload(x)
    y = backend.quant_matvec(w, xb)
    got = backend.download(y)
    assert got.shape == (rows,)
    y64 = oracle.matvec_f64(qt.id, blob, rows, cols, x)
    assert rel_err(got, y64) <= TOL
    # the engine's fp32 accumulation is far tighter than the bar; a layout or scale bug is not
    assert rel_err(got, y64) <= 1e-5
    yref = oracle.matvec(qt.id, blob, rows, cols, x)  # the reference's float loop
    assert rel_err(got, yref.astype(np.float64)) <= TOL
    # linearity: scaling x by 2 scales every product and partial sum exactly
    x2 = backend.upload(2.0 * x)
    y2 = backend.quant_matvec(w, x2)
    assert np.array_equal(bits(backend.download(y2)), bits(2.0 * got))
    for b in (xb, y, x2, y2):
        backend.release(b)


@pytest.mark.parametrize("qt", FORMATS, ids=lambda q: q.name)
def test_gemv_add_and_batch(backend, uploaded, qt):
    rows, cols = SHAPES[qt][2]
    note("add+batch", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    B = 3
    xs = S.activations_f32(99, B * cols).reshape(B, cols)
    add = S.activations_f32(98, rows)
    singles = []
    for b in range(B):
        xb = backend.upload(xs[b])
        y = backend.quant_matvec(w, xb)
        singles.append(backend.download(y))
        backend.release(y)
        # quantMatvecAdd: y = fl(W.x) + add, the add rounded on its own
        ab = backend.upload(add)
        ya = backend.quant_matvec_add(w, xb, ab)
        assert np.array_equal(bits(backend.download(ya)), bits(singles[-1] + add))
        for h in (ab, ya, xb):
            backend.release(h)
    xbb = backend.upload(xs, shape=(B, cols))
    yb = backend.quant_matvec(w, xbb)
    assert yb.shape == (B, rows)
    got = backend.download(yb).reshape(B, rows)
    # B >= 3 may run on the matrix cores (a different fp32 summation order than B = 1)
    for b in range(B):
        assert rel_err(got[b], singles[b].astype(np.float64)) <= 1e-5
        assert rel_err(got[b], oracle.matvec_f64(qt.id, blob, rows, cols, xs[b])) <= TOL
    backend.release(yb)
    backend.release(xbb)


# Batched GEMV shapes the matrix-core kernel takes (K <= 4096, K % 128 == 0), plus the
# benchmark's batch-8 Q4_0 shape; rows not a multiple of 16 exercise the last tile.
BATCH_CASES = [
    (QuantType.Q4_0, 300, 1024), (QuantType.Q4_0, 11008, 4096),
    (QuantType.Q8_0, 300, 1024), (QuantType.Q8_0, 4096, 4096),
    (QuantType.Q4_K, 300, 2304), (QuantType.Q4_K, 1024, 4096),
    (QuantType.Q6_K, 300, 2304), (QuantType.Q6_K, 2000, 4096),
]


@pytest.mark.parametrize("qt,rows,cols", BATCH_CASES, ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [3, 8, 9, 16, 21])
def test_gemv_batched_matches_oracle(backend, uploaded, qt, rows, cols, B):
    note("batched", qt.name, rows, cols, "B", B)
    blob, w = uploaded(qt, rows, cols)
    xs = S.activations_f32(rows + 7 * B, B * cols).reshape(B, cols)
    add = S.activations_f32(rows + 5, B * rows).reshape(B, rows)
    xb = backend.upload(xs, shape=(B, cols))
    ab = backend.upload(add, shape=(B, rows))
    y = backend.quant_matvec(w, xb)
    ya = backend.quant_matvec_add(w, xb, ab)
    got = backend.download(y).reshape(B, rows)
    gota = backend.download(ya).reshape(B, rows)
    for b in range(B):
        y64 = oracle.matvec_f64(qt.id, blob, rows, cols, xs[b])
        assert rel_err(got[b], y64) <= TOL, f"row {b}"
        assert rel_err(got[b], y64) <= 1e-5, f"row {b}"
    # quantMatvecAdd rounds the add on its own
    assert np.array_equal(bits(gota), bits(got + add))
    # each batch row depends on its own x only: a permuted batch gives the permuted rows.
    # Rows are launched in groups of up to 16 (a remainder of 1-2 rows takes the vector-ALU
    # kernel, which sums in another order), so the permutation stays inside each group.
    perm = np.arange(B)
    for c in range(0, B, 16):
        if min(B, c + 16) - c >= 3:
            perm[c:c + 16] = np.roll(perm[c:c + 16], 1)
    xp = backend.upload(np.ascontiguousarray(xs[perm]), shape=(B, cols))
    yp = backend.quant_matvec(w, xp)
    assert np.array_equal(bits(backend.download(yp).reshape(B, rows)), bits(got[perm]))
    # scaling x by 2 scales every product and partial sum exactly
    x2 = backend.upload(2.0 * xs, shape=(B, cols))
    y2 = backend.quant_matvec(w, x2)
    assert np.array_equal(bits(backend.download(y2).reshape(B, rows)), bits(2.0 * got))
    for h in (xb, ab, y, ya, xp, yp, x2, y2):
        backend.release(h)


# Up to 8 rows, Q4_K and Q6_K run rounds of 4 tiles, and a launch whose workgroups hold at
# least one full round takes the tile loop without skip paths (every slot's loads on every
# path, the compute behind the tile test). 28672 + 48 rows give 1795 tiles: 7 or 8 per
# workgroup on a 256-CU device, the last round partial; Q6_K 4096 x 14336 runs four column
# windows of 64 workgroups and 4 tiles each. Checked against the oracle row by row, and
# bit-identical under a batch permutation and an exact scaling of x.
@pytest.mark.parametrize("qt,rows,cols", [(QuantType.Q4_K, 28672 + 48, 4096), (QuantType.Q6_K, 4096, 14336)],
                         ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [4, 8])
def test_gemv_batched_full_rounds_match_oracle(backend, qt, rows, cols, B):
    note("batched full rounds", qt.name, rows, cols, "B", B)
    blob = S.quant_blocks(qt, 0x5A0 + rows, rows, cols)
    w = backend.upload_quantized(blob, qt, (rows, cols))
    xs = S.activations_f32(rows + 11 * B, B * cols).reshape(B, cols)
    xb = backend.upload(xs, shape=(B, cols))
    y = backend.quant_matvec(w, xb)
    got = backend.download(y).reshape(B, rows)
    for b in range(B):
        y64 = oracle.matvec_f64(qt.id, blob, rows, cols, xs[b])
        assert rel_err(got[b], y64) <= 4e-5, f"row {b}"
    perm = np.roll(np.arange(B), 1)
    xp = backend.upload(np.ascontiguousarray(xs[perm]), shape=(B, cols))
    yp = backend.quant_matvec(w, xp)
    assert np.array_equal(bits(backend.download(yp).reshape(B, rows)), bits(got[perm]))
    x2 = backend.upload(2.0 * xs, shape=(B, cols))
    y2 = backend.quant_matvec(w, x2)
    assert np.array_equal(bits(backend.download(y2).reshape(B, rows)), bits(2.0 * got))
    for h in (w, xb, y, xp, yp, x2, y2):
        backend.release(h)


# K above one 4096-column launch window: the batched kernel runs equal windows, each adding
# the previous window's y, and the caller's add joins only in the last one (11008 = three
# windows of 116, 116 and 112 blocks; 14336 = four of 112).
# K = 11008 for the K-quants gives 344 blocks in three windows that must start on
# superblocks (120-block windows, not 116)
WIDE_CASES = [
    (QuantType.Q4_0, 700, 11008), (QuantType.Q8_0, 300, 8192),
    (QuantType.Q4_K, 300, 12288), (QuantType.Q6_K, 512, 14336),
    (QuantType.Q4_K, 200, 11008), (QuantType.Q6_K, 136, 11008),
]


@pytest.mark.parametrize("qt,rows,cols", WIDE_CASES, ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [3, 8, 16])
def test_gemv_batched_wide_k(backend, uploaded, qt, rows, cols, B):
    note("batched wide", qt.name, rows, cols, "B", B)
    blob, w = uploaded(qt, rows, cols)
    xs = S.activations_f32(rows + 11 * B, B * cols).reshape(B, cols)
    add = S.activations_f32(rows + 13, B * rows).reshape(B, rows)
    xb = backend.upload(xs, shape=(B, cols))
    ab = backend.upload(add, shape=(B, rows))
    y = backend.quant_matvec(w, xb)
    ya = backend.quant_matvec_add(w, xb, ab)
    got = backend.download(y).reshape(B, rows)
    gota = backend.download(ya).reshape(B, rows)
    # The matrix-core sums of one block round in one direction (a bias of a fraction of an
    # fp32 ulp of the block's largest product, times its scale d > 0), so the error grows
    # with the number of blocks: 1.0e-5 measured for Q4_0 at K = 11008. The bound stays 25x
    # inside the decode tolerance TOL.
    for b in range(B):
        y64 = oracle.matvec_f64(qt.id, blob, rows, cols, xs[b])
        assert rel_err(got[b], y64) <= 4e-5, f"row {b}"
    assert np.array_equal(bits(gota), bits(got + add))
    for h in (xb, ab, y, ya):
        backend.release(h)


# 9-16 batch rows over K = 4096 run two 2048-column windows, each in its own workgroups, and
# sum_windows_kernel adds their sums in window order: y equals, bit for bit, fl(y_left +
# y_right) of the two column halves uploaded as matrices of their own (one window each, the
# same waves' slices of x), and the add joins on its own. The row counts give 19 to 2500
# tiles: one to ten per workgroup, partial rounds and the ring's second slot empty.
HALVES_CASES = [
    (QuantType.Q8_0, 300), (QuantType.Q4_K, 4096), (QuantType.Q4_K, 6144), (QuantType.Q4_0, 11008),
    (QuantType.Q6_K, 11008), (QuantType.Q4_K, 28672 + 48), (QuantType.Q8_0, 28672 + 48), (QuantType.Q4_K, 40000),
]


@pytest.mark.parametrize("qt,rows", HALVES_CASES, ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [9, 16])
def test_gemv_batched_two_windows_equal_sum_of_halves(backend, qt, rows, B):
    cols, half = 4096, 2048
    note("batched halves", qt.name, rows, cols, "B", B)
    blob = S.quant_blocks(qt, 0x4A1F + rows, rows, cols)
    per_row = cols // qt.block_elements * qt.block_bytes
    grid = np.frombuffer(blob, dtype=np.uint8).reshape(rows, per_row)
    left = np.ascontiguousarray(grid[:, : per_row // 2]).tobytes()
    right = np.ascontiguousarray(grid[:, per_row // 2:]).tobytes()
    w = backend.upload_quantized(blob, qt, (rows, cols))
    wl = backend.upload_quantized(left, qt, (rows, half))
    wr = backend.upload_quantized(right, qt, (rows, half))
    xs = S.activations_f32(rows + 3 * B, B * cols).reshape(B, cols)
    add = S.activations_f32(rows + 17, B * rows).reshape(B, rows)
    xb = backend.upload(xs, shape=(B, cols))
    xlb = backend.upload(np.ascontiguousarray(xs[:, :half]), shape=(B, half))
    xrb = backend.upload(np.ascontiguousarray(xs[:, half:]), shape=(B, half))
    ab = backend.upload(add, shape=(B, rows))
    y, ya = backend.quant_matvec(w, xb), backend.quant_matvec_add(w, xb, ab)
    yl, yr = backend.quant_matvec(wl, xlb), backend.quant_matvec(wr, xrb)
    got = backend.download(y).reshape(B, rows)
    halves = backend.download(yl).reshape(B, rows) + backend.download(yr).reshape(B, rows)
    assert np.array_equal(bits(got), bits(halves))
    assert np.array_equal(bits(backend.download(ya).reshape(B, rows)), bits(got + add))
    y64 = oracle.matvec_f64(qt.id, blob, rows, cols, xs[B - 1])
    assert rel_err(got[B - 1], y64) <= 4e-5
    for h in (w, wl, wr, xb, xlb, xrb, ab, y, ya, yl, yr):
        backend.release(h)


@pytest.mark.parametrize("cols", [4096, 11008])
@pytest.mark.parametrize("B", [8, 16])
@pytest.mark.parametrize("shift", [0, 1])
def test_gemv_batched_add_in_place(backend, uploaded, cols, B, shift):
    """quantMatvecAdd with y on the add buffer itself (a residual updated in place). The
    column windows' partial sums meet in a workspace and one kernel adds them and then add,
    element by element, so the in-place call runs the same launches as the out-of-place one
    and gives the same bits. shift = 1 puts y 4 bytes past a 16-byte boundary (the window
    sums then take their one-element path)."""
    qt, rows = QuantType.Q4_0, 1000
    note("batched in-place add", qt.name, rows, cols, "B", B, "shift", shift)
    blob, w = uploaded(qt, rows, cols)
    xs = S.activations_f32(rows + 3, B * cols).reshape(B, cols)
    add = S.activations_f32(rows + 4, B * rows).reshape(B, rows)
    xb = backend.upload(xs, shape=(B, cols))
    ab = backend.upload(add, shape=(B, rows))
    ref = backend.download(backend.quant_matvec_add(w, xb, ab)).reshape(B, rows)
    res = backend.upload(np.concatenate([np.zeros(shift, np.float32), add.reshape(-1)]))
    rp = backend.buffer_desc(res).device_ptr + 4 * shift
    backend.quant_matvec_into(w, backend.buffer_desc(xb).device_ptr, rp, rp, B)
    backend.sync()
    got = backend.download(res)[shift:].reshape(B, rows)
    assert np.array_equal(bits(got), bits(ref))
    for b in range(B):
        y64 = oracle.matvec_f64(qt.id, blob, rows, cols, xs[b]) + add[b].astype(np.float64)
        assert rel_err(got[b], y64) <= 4e-5, f"row {b}"
    for h in (xb, ab, res):
        backend.release(h)


@pytest.mark.parametrize("qt", [QuantType.Q4_0, QuantType.Q8_0, QuantType.Q4_K, QuantType.Q6_K], ids=lambda q: q.name)
def test_gemv_batched_one_hot_and_range(backend, uploaded, qt):
    rows, cols = (300, 2304) if qt in (QuantType.Q4_K, QuantType.Q6_K) else (300, 1024)
    note("batched onehot/range", qt.name, rows, cols)
    blob, w = uploaded(qt, rows, cols)
    wd = oracle.dequant_matrix(qt.id, blob, rows, cols)
    B = 5
    js = [0, 31, cols // 2 + 3, cols - 1, 17]
    xs = np.zeros((B, cols), np.float32)
    for b, j in enumerate(js):
        xs[b, j] = 1.0
    xb = backend.upload(xs, shape=(B, cols))
    y = backend.quant_matvec(w, xb)
    got = backend.download(y).reshape(B, rows)
    for b, j in enumerate(js):
        assert np.array_equal(got[b], wd[:, j]), f"column {j}"
    backend.release(y)
    backend.release(xb)
    # x far outside fp16 range, and far below it: the per-row power-of-two scale keeps the
    # hi/lo split exact to 22 bits either way. Slice maxima of 2^118 and more (x near 1e36)
    # need the 2^(24 - e) undo factor applied in two parts; the batch then agrees with the
    # vector-ALU kernel's B = 1 results instead of turning into inf or NaN.
    scales = np.array([1e30, 1e-30, 1.0, 3e4, 1e-6, 1e36, 5e35], np.float32)
    B = len(scales)
    xs = S.activations_f32(4242, B * cols).reshape(B, cols)
    xr = (xs * scales[:, None]).astype(np.float32)
    xb = backend.upload(xr, shape=(B, cols))
    y = backend.quant_matvec(w, xb)
    got = backend.download(y).reshape(B, rows)
    assert np.isfinite(got).all()
    for b in range(B):
        assert rel_err(got[b], oracle.matvec_f64(qt.id, blob, rows, cols, xr[b])) <= 1e-5, f"scale {scales[b]}"
        x1 = backend.upload(xr[b])
        y1 = backend.quant_matvec(w, x1)
        assert rel_err(got[b], backend.download(y1).astype(np.float64)) <= 1e-5, f"B=1 vs batch, scale {scales[b]}"
        backend.release(y1)
        backend.release(x1)
    backend.release(y)
    backend.release(xb)


def test_shape_and_index_errors(backend, uploaded):
    blob, w = uploaded(QuantType.Q4_0, 13, 96)
    bad = backend.upload(np.zeros(95, np.float32))
    with pytest.raises(IllegalArgumentException, match="shape mismatch"):
        backend.quant_matvec(w, bad)
    backend.release(bad)
    with pytest.raises(IllegalArgumentException, match="out of range"):
        backend.quant_gather_row(w, 13)
    with pytest.raises(IllegalArgumentException, match="out of range"):
        backend.quant_gather_row(w, -1)
    x = backend.upload(np.zeros(96, np.float32))
    short = backend.upload(np.zeros(12, np.float32))
    with pytest.raises(IllegalArgumentException, match="add"):
        backend.quant_matvec_add(w, x, short)
    backend.release(x)
    backend.release(short)


def test_device_generator_matches_host(backend):
    import ctypes as C

    from jax4j_amd import _native as N

    lib = N.load()
    for qt, rows, cols in ((QuantType.Q4_K, 7, 512), (QuantType.Q6_K, 5, 768), (QuantType.Q8_0, 9, 96), (QuantType.Q4_0, 3, 64)):
        note("synth", qt.name)
        nbytes = qt.byte_size_for(rows * cols)
        host = S.quant_blocks(qt, 1234, rows, cols)
        buf = backend.upload(np.zeros((nbytes + 3) // 4, np.float32))
        ptr = backend.buffer_desc(buf).device_ptr
        assert lib.j4q_synth_quant_device(qt.id, 1234, rows, cols, C.c_void_p(ptr), nbytes, None) == 0
        backend.sync()
        dev = backend.download(buf).view(np.uint8)[:nbytes]
        assert np.array_equal(dev, host)
        backend.release(buf)
    n = 4099
    buf = backend.upload(np.zeros(n, np.float32))
    assert lib.j4q_synth_f32_device(77, n, C.c_void_p(backend.buffer_desc(buf).device_ptr), None) == 0
    assert np.array_equal(bits(backend.download(buf)), bits(S.activations_f32(77, n)))
    backend.release(buf)


def test_concurrent_callers_get_serial_results(backend, uploaded):
    """The ABI is callable from many threads (pattern: VulkanExecutionTest.java:72-105)."""
    blob, w = uploaded(QuantType.Q4_K, 1024, 4096)
    xs = [S.activations_f32(500 + i, 4096) for i in range(8)]
    serial = []
    for x in xs:
        xb = backend.upload(x)
        y = backend.quant_matvec(w, xb)
        serial.append(backend.download(y))
        backend.release(y)
        backend.release(xb)
    results = [None] * len(xs)
    errors = []

    def work(i):
        try:
            xb = backend.upload(xs[i])
            y = backend.quant_matvec(w, xb)
            results[i] = backend.download(y)
            backend.release(y)
            backend.release(xb)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(xs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors
    for a, b in zip(results, serial):
        assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("qt", [QuantType.Q4_K, QuantType.Q6_K, QuantType.Q8_0], ids=lambda q: q.name)
@pytest.mark.parametrize("B", [1, 4])
def test_concat_rows_fused_gemv(backend, qt, B):
    """q/k/v-style fusion: one matrix over the parts' rows gives the parts' outputs bit for bit."""
    cols = 512
    shapes = [40, 24, 24]
    note("concat", qt.name, shapes, cols, "B", B)
    blobs = [S.quant_blocks(qt, 300 + i, r, cols) for i, r in enumerate(shapes)]
    parts = [backend.upload_quantized(b, qt, (r, cols)) for b, r in zip(blobs, shapes)]
    fused = backend.concat_rows(parts)
    assert fused.shape == (sum(shapes), cols)
    assert np.array_equal(backend.export_quantized(fused), np.concatenate(blobs))
    xs = S.activations_f32(77 + B, B * cols).reshape(B, cols)
    xb = backend.upload(xs if B > 1 else xs[0], shape=(B, cols) if B > 1 else None)
    yf = backend.download(backend.quant_matvec(fused, xb)).reshape(B, -1)
    off = 0
    for p, r in zip(parts, shapes):
        yp = backend.download(backend.quant_matvec(p, xb)).reshape(B, r)
        assert np.array_equal(bits(yf[:, off:off + r]), bits(yp))
        off += r
    with pytest.raises(IllegalArgumentException):
        other = backend.upload_quantized(S.quant_blocks(QuantType.Q4_0, 5, 8, cols), QuantType.Q4_0, (8, cols))
        backend.concat_rows([parts[0], other])


# K of any block-aligned width (CpuQ4Gemm.java:26-46,79-83; CpuBackend.java:712-714): up to
# 32768 columns one vector-ALU launch holds x in LDS (15360 was the previous image size,
# 15488 the first K past it); wider K runs as equal column windows chained through the
# previous window's y (40960 = two windows of 20480, 53248 = two of 26624). B >= 3 runs the
# matrix-core kernel in 4096-column windows.
WIDEK_CASES = [
    (QuantType.Q4_0, 96, 15360), (QuantType.Q4_0, 96, 15488), (QuantType.Q4_0, 80, 28672),
    (QuantType.Q8_0, 64, 32768), (QuantType.Q8_0, 40, 40960),
    (QuantType.Q4_K, 72, 28672), (QuantType.Q4_K, 40, 53248),
    (QuantType.Q6_K, 64, 32768), (QuantType.Q6_K, 40, 40960),
    (QuantType.Q2_0, 48, 28672), (QuantType.Q2_0, 24, 40960),
]


@pytest.mark.parametrize("qt,rows,cols", WIDEK_CASES, ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [1, 2, 3, 16])
def test_gemv_any_k(backend, uploaded, qt, rows, cols, B):
    if B >= 3 and qt == QuantType.Q2_0:
        B = 4  # Q2_0 has no matrix-core path: 4 vector-ALU passes
    note("any-k", qt.name, rows, cols, "B", B)
    blob, w = uploaded(qt, rows, cols)
    xs = S.activations_f32(cols + 17 * B, B * cols).reshape(B, cols)
    add = S.activations_f32(cols + 19, B * rows).reshape(B, rows)
    xb = backend.upload(xs if B > 1 else xs[0], shape=(B, cols) if B > 1 else None)
    ab = backend.upload(add if B > 1 else add[0], shape=(B, rows) if B > 1 else None)
    y = backend.quant_matvec(w, xb)
    ya = backend.quant_matvec_add(w, xb, ab)
    got = backend.download(y).reshape(B, rows)
    gota = backend.download(ya).reshape(B, rows)
    ref = oracle.matmul_f64(qt.id, blob, rows, cols, xs)
    # fp32 accumulation over one launch or several chained windows: 1e-5 (the vector-ALU
    # kernel) and 1e-4 for the matrix-core kernel, whose block sums round one way (the bias
    # grows with the number of blocks; both far inside the 1e-3 decode tolerance)
    bound = 1e-5 if B < 3 or qt == QuantType.Q2_0 else 1e-4
    for b in range(B):
        assert rel_err(got[b], ref[b]) <= bound, f"row {b}"
    # the caller's add joins only after the last window, rounded on its own
    assert np.array_equal(bits(gota), bits(got + add))
    for h in (xb, ab, y, ya):
        backend.release(h)


# Batch rows of 1-2 over 8193..15360 columns (one 16-wave workgroup per CU, a 480-chunk x
# image): rows below one workgroup's 16 and not a multiple of it, a partial last step
# (K = 9024: 26 chunks in the last step of 64) and 40000 rows (ten per wave). Checked
# against the fp64 oracle, bit-identical on repeated calls and under an exact scaling of x,
# the add rounded on its own, and y updated in place on the add buffer.
WIDE_WINDOW_CASES = [
    (QuantType.Q6_K, 1, 14336), (QuantType.Q6_K, 13, 14336), (QuantType.Q6_K, 4096 + 5, 14336),
    (QuantType.Q4_K, 300, 9216), (QuantType.Q4_0, 700, 9024), (QuantType.Q8_0, 200, 15360),
    (QuantType.Q2_0, 100, 11008), (QuantType.Q6_K, 40000, 14336),
]


@pytest.mark.parametrize("qt,rows,cols", WIDE_WINDOW_CASES, ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [1, 2])
def test_gemv_wide_window_b1(backend, qt, rows, cols, B):
    note("wide window", qt.name, rows, cols, "B", B)
    blob = S.quant_blocks(qt, 0x57E9 + rows + cols, rows, cols)
    w = backend.upload_quantized(blob, qt, (rows, cols))
    xs = S.activations_f32(rows + 23 * B, B * cols).reshape(B, cols)
    add = S.activations_f32(rows + 29, B * rows).reshape(B, rows)
    shape_x, shape_y = ((B, cols), (B, rows)) if B > 1 else (None, None)
    xb = backend.upload(xs if B > 1 else xs[0], shape=shape_x)
    ab = backend.upload(add if B > 1 else add[0], shape=shape_y)
    y, y2 = backend.quant_matvec(w, xb), backend.quant_matvec(w, xb)
    ya = backend.quant_matvec_add(w, xb, ab)
    got = backend.download(y).reshape(B, rows)
    ref = oracle.matmul_f64(qt.id, blob, rows, cols, xs)
    for b in range(B):
        assert rel_err(got[b], ref[b]) <= 1e-5, f"row {b}"
    assert np.array_equal(bits(backend.download(y2).reshape(B, rows)), bits(got))
    assert np.array_equal(bits(backend.download(ya).reshape(B, rows)), bits(got + add))
    xd = backend.upload(2.0 * xs if B > 1 else 2.0 * xs[0], shape=shape_x)
    yd = backend.quant_matvec(w, xd)
    assert np.array_equal(bits(backend.download(yd).reshape(B, rows)), bits(2.0 * got))
    res = backend.upload(add.reshape(-1))
    rp = backend.buffer_desc(res).device_ptr
    backend.quant_matvec_into(w, backend.buffer_desc(xb).device_ptr, rp, rp, B)
    backend.sync()
    assert np.array_equal(bits(backend.download(res).reshape(B, rows)), bits(got + add))
    for h in (w, xb, ab, y, y2, ya, xd, yd, res):
        backend.release(h)


# J4Q_GEMV_FP32: batched GEMV runs every row on the batch-1 kernel (fp32 x, fp32 accumulation,
# no matrix cores), so each row equals quantMatvec of that row alone bit for bit, with the add
# on its own and in place; B = 3 and 17 would otherwise take the matrix cores (17: a 16-row
# launch and a remainder). K = 40960 runs chained column windows.
@pytest.mark.parametrize("qt,rows,cols", [(QuantType.Q4_K, 300, 4096), (QuantType.Q6_K, 200, 14336),
                                          (QuantType.Q4_0, 257, 4096), (QuantType.Q8_0, 64, 40960)],
                         ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [3, 17])
def test_gemv_fp32_policy_rows_equal_single_calls(backend, qt, rows, cols, B):
    note("fp32 policy", qt.name, rows, cols, "B", B)
    prev = backend.set_gemv_policy("fp32")
    handles = []
    try:
        blob = S.quant_blocks(qt, 0xF32 + rows + cols, rows, cols)
        w = backend.upload_quantized(blob, qt, (rows, cols))
        xs = S.activations_f32(rows + 31 * B, B * cols).reshape(B, cols)
        add = S.activations_f32(rows + 37, B * rows).reshape(B, rows)
        xb, ab = backend.upload(xs, shape=(B, cols)), backend.upload(add, shape=(B, rows))
        y, ya = backend.quant_matvec(w, xb), backend.quant_matvec_add(w, xb, ab)
        handles += [w, xb, ab, y, ya]
        got = backend.download(y).reshape(B, rows)
        for b in range(B):
            xr = backend.upload(xs[b])
            yr = backend.quant_matvec(w, xr)
            handles += [xr, yr]
            assert np.array_equal(bits(backend.download(yr)), bits(got[b])), f"row {b}"
        assert np.array_equal(bits(backend.download(ya).reshape(B, rows)), bits(got + add))
        assert rel_err(got[0], oracle.matvec_f64(qt.id, blob, rows, cols, xs[0])) <= 1e-5
        if cols <= 32768:
            res = backend.upload(add.reshape(-1))
            handles.append(res)
            rp = backend.buffer_desc(res).device_ptr
            backend.quant_matvec_into(w, backend.buffer_desc(xb).device_ptr, rp, rp, B)
            backend.sync()
            assert np.array_equal(bits(backend.download(res).reshape(B, rows)), bits(got + add))
    finally:
        backend.set_gemv_policy(prev)
        for h in handles:
            backend.release(h)


def test_in_place_add_wider_than_one_window_is_rejected(backend, uploaded):
    """An add that overlaps y is read after the first window rewrote y, so above 32768 columns
    the stream-ordered entry point refuses it (the SPI's quantMatvecAdd always returns a new
    buffer and is not affected)."""
    qt, rows, cols = QuantType.Q4_0, 24, 40960
    blob, w = uploaded(qt, rows, cols)
    x = backend.upload(S.activations_f32(5, cols))
    res = backend.upload(np.zeros(rows, np.float32))
    rp = backend.buffer_desc(res).device_ptr
    with pytest.raises(IllegalArgumentException, match="overlaps y"):
        backend.quant_matvec_into(w, backend.buffer_desc(x).device_ptr, rp, rp, 1)
    backend.release(x)
    backend.release(res)


def test_add_partly_overlapping_y_is_rejected(backend, uploaded):
    """An add that overlaps y without being y itself would be read by one thread while
    another rewrites it, so the stream-ordered entry point refuses it at any size."""
    qt, rows, cols = QuantType.Q4_0, 24, 512
    blob, w = uploaded(qt, rows, cols)
    x = backend.upload(S.activations_f32(6, 4 * cols))
    res = backend.upload(np.zeros(4 * rows + 4, np.float32))
    rp = backend.buffer_desc(res).device_ptr
    for B in (1, 4):
        with pytest.raises(IllegalArgumentException, match="without being y itself"):
            backend.quant_matvec_into(w, backend.buffer_desc(x).device_ptr, rp + 16, rp, B)
    backend.release(x)
    backend.release(res)


@pytest.mark.parametrize("qt,rows,cols", [(QuantType.Q4_0, 40, 40960), (QuantType.Q6_K, 40, 40960),
                                          (QuantType.Q4_K, 24, 53248)], ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("B", [17, 18, 33, 34])
def test_batched_in_place_add_above_one_window(backend, uploaded, qt, rows, cols, B):
    """A residual updated in place (add = y) at more than 16 batch rows over K > 32768: the
    rows past the last full 16 stay on the matrix cores (a 1-2 row remainder on the
    vector-ALU kernel would chain its column windows through y and read the add after the
    first window rewrote it). Bit for bit equal to the out-of-place quantMatvecAdd, which
    splits the batch the same way, and within the batched bound of the oracle."""
    note("in place above one window", qt.name, rows, cols, "B", B)
    blob, w = uploaded(qt, rows, cols)
    xs = S.activations_f32(cols + 3 * B, B * cols).reshape(B, cols)
    add = S.activations_f32(cols + 5 * B, B * rows).reshape(B, rows)
    xb = backend.upload(xs, shape=(B, cols))
    ab = backend.upload(add, shape=(B, rows))
    ya = backend.quant_matvec_add(w, xb, ab)
    want = backend.download(ya).reshape(B, rows)
    res = backend.upload(add, shape=(B, rows))
    rp = backend.buffer_desc(res).device_ptr
    backend.quant_matvec_into(w, backend.buffer_desc(xb).device_ptr, rp, rp, B)
    backend.sync()
    got = backend.download(res).reshape(B, rows)
    assert np.array_equal(bits(got), bits(want))
    ref = oracle.matmul_f64(qt.id, blob, rows, cols, xs) + add.astype(np.float64)
    for b in range(B):
        assert rel_err(got[b], ref[b]) <= 1e-4, f"row {b}"
    for h in (xb, ab, ya, res):
        backend.release(h)

"""Pins the CPU oracle (oracle/quant_ref.c) before anything is checked against it.

The reference ships no golden vectors for this path, so each oracle function is pinned by
checks a plausible mistake cannot pass: exhaustive comparison with a library routine
(numpy.float16), hand-derived known answers (tests/golden/kat_blocks.json, built from the
block layouts with exact power-of-two scales), an independently written vectorised numpy
decoder per format, invariants (one-hot x returns a column exactly; fp64 brute force),
and the reference's sequential accumulation order for Q4_0 (CpuQ4Gemm.java:29-45).
"""
from __future__ import annotations

import json
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import oracle
from jax4j_amd import QuantType
from jax4j_amd import synthetic as S

KAT = json.loads((Path(__file__).parent / "golden" / "kat_blocks.json").read_text())["cases"]
FORMATS = [QuantType.Q4_0, QuantType.Q8_0, QuantType.Q4_K, QuantType.Q6_K, QuantType.Q2_0]


# ---- independent numpy decoders, written from the published block layouts ---------------

def _f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32).reshape(-1)


def np_dequant(qt: QuantType, blob: np.ndarray, rows: int, cols: int) -> np.ndarray:
    blk = blob.reshape(-1, qt.block_bytes)
    nb = blk.shape[0]
    if qt == QuantType.Q8_0:
        d = _f16(blk[:, 0:2])
        w = d[:, None] * blk[:, 2:].view(np.int8).astype(np.float32)
    elif qt == QuantType.Q4_0:
        d = _f16(blk[:, 0:2])
        qs = blk[:, 2:].astype(np.int32)
        codes = np.concatenate([qs & 15, qs >> 4], axis=1) - 8
        w = d[:, None] * codes.astype(np.float32)
    elif qt == QuantType.Q2_0:
        d = _f16(blk[:, 0:2])
        qs = blk[:, 2:].astype(np.int32)
        codes = np.stack([(qs >> (2 * s)) & 3 for s in range(4)], axis=2).reshape(nb, 128) - 1
        w = d[:, None] * codes.astype(np.float32)
    elif qt == QuantType.Q4_K:
        d, dmin = _f16(blk[:, 0:2]), _f16(blk[:, 2:4])
        s = blk[:, 4:16].astype(np.int32)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], axis=1)
        mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        qs = blk[:, 16:].astype(np.int32).reshape(nb, 4, 32)
        codes = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32)
        d1 = (d[:, None] * sc.astype(np.float32))[:, :, None]
        m1 = (dmin[:, None] * mn.astype(np.float32))[:, :, None]
        w = (d1 * codes.astype(np.float32) - m1).reshape(nb, 256)
    elif qt == QuantType.Q6_K:
        ql = blk[:, 0:128].astype(np.int32).reshape(nb, 2, 64)
        qh = blk[:, 128:192].astype(np.int32).reshape(nb, 2, 32)
        sc = blk[:, 192:208].view(np.int8).astype(np.float32)
        d = _f16(blk[:, 208:210])
        lo, hi = ql[:, :, :32], ql[:, :, 32:]
        q = np.concatenate(
            [
                (lo & 15) | ((qh & 3) << 4),
                (hi & 15) | (((qh >> 2) & 3) << 4),
                (lo >> 4) | (((qh >> 4) & 3) << 4),
                (hi >> 4) | (((qh >> 6) & 3) << 4),
            ],
            axis=2,
        ).reshape(nb, 256) - 32
        scale = d[:, None] * sc[:, np.arange(256) // 16]
        w = scale * q.astype(np.float32)
    else:
        raise AssertionError(qt)
    return w.reshape(rows, cols).astype(np.float32)


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---- binary16 ---------------------------------------------------------------------------

def test_half_to_float_exhaustive_against_numpy():
    patterns = np.arange(65536, dtype=np.uint16)
    ours = oracle.half_to_float_array(patterns)
    ref = patterns.view(np.float16).astype(np.float32)
    assert np.array_equal(bits(ours), bits(ref))
    # the scalar entry point agrees on every non-NaN pattern (NaNs are quieted by ctypes)
    lib = oracle.load()
    for b in (0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x7C00, 0x8001, 0xFC00):
        assert np.float32(lib.ref_half_to_float(b)) == ref[b]


# ---- hand-derived known answers ---------------------------------------------------------

@pytest.mark.parametrize("case", KAT, ids=[c["name"] for c in KAT])
def test_kat_dequant_exact(case):
    blob = np.frombuffer(bytes.fromhex(case["blob_hex"]), dtype=np.uint8)
    got = oracle.dequant_matrix(case["type_id"], blob, case["rows"], case["cols"]).reshape(-1)
    assert np.array_equal(bits(got), bits(np.array(case["values"], dtype=np.float32)))


@pytest.mark.parametrize("case", KAT, ids=[c["name"] for c in KAT])
def test_kat_gemv_exact(case):
    blob = np.frombuffer(bytes.fromhex(case["blob_hex"]), dtype=np.uint8)
    k = case["cols"]
    ones = np.ones(k, dtype=np.float32)
    ramp = ((np.arange(k) % 7) - 3).astype(np.float32)
    assert oracle.matvec(case["type_id"], blob, 1, k, ones)[0] == np.float32(case["gemv_x_ones"])
    assert oracle.matvec(case["type_id"], blob, 1, k, ramp)[0] == np.float32(case["gemv_x_ramp"])


# ---- independent decoder, invariants -----------------------------------------------------

@pytest.mark.parametrize("qt", FORMATS, ids=lambda q: q.name)
def test_dequant_matches_independent_numpy_decoder(qt):
    rows, cols = 37, 4 * max(qt.block_elements, 256)
    blob = S.quant_blocks(qt, 0x5EED5, rows, cols)
    ref = np_dequant(qt, blob, rows, cols)
    got = oracle.dequant_matrix(qt.id, blob, rows, cols)
    assert np.array_equal(bits(got), bits(ref))
    for r in (0, 17, rows - 1):
        assert np.array_equal(bits(oracle.gather_row(qt.id, blob, r, rows, cols)), bits(ref[r]))


@pytest.mark.parametrize("qt", FORMATS, ids=lambda q: q.name)
def test_onehot_x_returns_column_exactly(qt):
    rows, cols = 19, 2 * max(qt.block_elements, 256)
    blob = S.quant_blocks(qt, 7, rows, cols)
    w = np_dequant(qt, blob, rows, cols)
    for j in (0, 1, 17, cols // 2 + 5, cols - 1):
        x = np.zeros(cols, dtype=np.float32)
        x[j] = 1.0
        y = oracle.matvec(qt.id, blob, rows, cols, x)
        assert np.array_equal(y, w[:, j])  # values: a -0.0 weight sums to +0.0
        assert np.array_equal(bits(y), bits(w[:, j] + np.float32(0.0)))


@pytest.mark.parametrize("qt", FORMATS, ids=lambda q: q.name)
def test_float_path_close_to_fp64_brute_force(qt):
    rows, cols = 64, 4096
    blob = S.quant_blocks(qt, 11, rows, cols)
    x = S.activations_f32(12, cols)
    y = oracle.matvec(qt.id, blob, rows, cols, x).astype(np.float64)
    y64 = oracle.matvec_f64(qt.id, blob, rows, cols, x)
    w = np_dequant(qt, blob, rows, cols).astype(np.float64)
    assert np.allclose(y64, w @ x.astype(np.float64), rtol=0, atol=1e-9 * np.abs(y64).max())
    assert np.abs(y - y64).max() <= 1e-5 * np.abs(y64).max()


def test_q4_0_follows_reference_sequential_order():
    """CpuQ4Gemm.multiply sums (d*(lo-8))*x[p] then (d*(hi-8))*x[p+16] for p = 0..15 per
    block, one float accumulator per row. A natural-order sum differs in the last bits."""
    rows, cols = 48, 1024
    blob = S.quant_blocks(QuantType.Q4_0, 3, rows, cols)
    x = S.activations_f32(4, cols)
    w = np_dequant(QuantType.Q4_0, blob, rows, cols)
    order = np.array([b * 32 + p + 16 * half for b in range(cols // 32) for p in range(16) for half in (0, 1)])
    terms = (w[:, order] * x[order]).astype(np.float32)  # each product rounded to float
    seq = np.add.accumulate(terms, axis=1, dtype=np.float32)[:, -1]
    natural = np.add.accumulate((w * x).astype(np.float32), axis=1, dtype=np.float32)[:, -1]
    got = oracle.q4_0_multiply(blob, rows, cols, x)
    assert np.array_equal(bits(got), bits(seq))
    assert not np.array_equal(bits(got), bits(natural))


def test_q4_0_reference_rejects_bad_dimensions_and_rows():
    lib = oracle.load()
    y = np.zeros(4, dtype=np.float32)
    x = np.zeros(64, dtype=np.float32)
    blob = np.zeros(4 * 2 * 18, dtype=np.uint8)
    p = oracle._p
    assert lib.ref_q4_0_multiply(p(y), p(x), p(blob), 4, 63) != 0  # cols % 32 != 0
    assert lib.ref_q4_0_multiply(p(y), p(x), p(blob), 0, 64) != 0  # rows <= 0
    assert lib.ref_q4_0_gather(p(x), p(blob), 4, 4, 64) != 0  # row == rows
    assert lib.ref_q4_0_gather(p(x), p(blob), -1, 4, 64) != 0


def test_geometry_table_matches_quant_type_enum():
    lib = oracle.load()
    import ctypes as C

    for qt in FORMATS:
        be, bb = C.c_int(), C.c_int()
        assert lib.ref_block_geometry(qt.id, C.byref(be), C.byref(bb)) == 0
        assert (be.value, bb.value) == (qt.block_elements, qt.block_bytes)
    assert lib.ref_block_geometry(3, None, None) != 0


# ---- activation quantizer and GEMM references ---------------------------------------------

def _bf16(v: np.ndarray) -> np.ndarray:
    """fp32 values that are exact in bf16 -> bf16 bit patterns."""
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    assert np.all((u & 0xFFFF) == 0)
    return (u >> 16).astype(np.uint16)


def test_quantize_act_closed_forms():
    k = 128
    x = np.zeros((1, k), dtype=np.float32)
    x[0, 0:32] = 3.0  # constant block: s = 3/127, every q = 127
    x[0, 32:64] = 0.0  # zero block: s = 0, q = 0
    x[0, 64:96] = np.arange(32, dtype=np.float32) - 15.0  # amax 16
    x[0, 96] = -127.0 / 8  # amax 127/8 -> s = 1/8 exactly, q = 8x
    x[0, 97:128] = np.float32(0.5)
    q, s = oracle.quantize_act(_bf16(x), 1, k)
    assert s[0, 0] == np.float32(3.0) / np.float32(127.0) and np.all(q[0, 0:32] == 127)
    assert s[0, 1] == 0.0 and np.all(q[0, 32:64] == 0)
    assert s[0, 3] == np.float32(0.125)
    assert q[0, 96] == -127 and np.all(q[0, 97:128] == 4)
    # block 2: s = 16/127, q = round_half_away(x * (1/s)) in float32
    s2 = np.float32(16.0) / np.float32(127.0)
    inv = np.float32(1.0) / s2
    prod = (x[0, 64:96] * inv).astype(np.float32)
    want = np.sign(prod) * np.floor(np.abs(prod) + np.float32(0.5))
    assert s[0, 2] == s2 and np.array_equal(q[0, 64:96], want.astype(np.int8))


def test_gemm_references_against_exact_integer_arithmetic():
    m, n, k = 5, 7, 256
    w_blob = S.quant_blocks(QuantType.Q8_0, 21, n, k)
    xb = S.activations_bf16(22, m * k).reshape(m, k)
    xq, xs = oracle.quantize_act(xb, m, k)
    nb = k // 32
    blk = w_blob.reshape(n, nb, 34)
    wq = blk[:, :, 2:].view(np.int8).astype(np.int64)
    wd = _f16(blk[:, :, 0:2]).reshape(n, nb)
    dots = np.einsum("mbk,nbk->mnb", xq.astype(np.int64).reshape(m, nb, 32), wq)
    scale = (xs[:, None, :] * wd[None, :, :]).astype(np.float32)
    # acc = fma(dot, s, acc) per block in order: the product and sum are formed exactly
    # (rationals) and rounded once to float32, ties to even
    want = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            acc = np.float32(0.0)
            for b in range(nb):
                acc = _f32_rne(Fraction(int(dots[i, j, b])) * Fraction(float(scale[i, j, b])) + Fraction(float(acc)))
            want[i, j] = acc
    got = oracle.gemm_int8_emulated(xq, xs, w_blob, m, n, k)
    assert np.array_equal(bits(got), bits(want))
    # four contiguous ranges of whole 4-block stages (8 blocks = 2 stages: one stage each for
    # ranges 0 and 1, none for 2 and 3), each folded from 0, partials added in order
    want4 = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            part = [np.float32(0.0)] * 4
            for b in range(nb):
                p = b // 4
                part[p] = _f32_rne(Fraction(int(dots[i, j, b])) * Fraction(float(scale[i, j, b])) + Fraction(float(part[p])))
            acc = part[0]
            for p in range(1, 4):
                acc = _f32_rne(Fraction(float(acc)) + Fraction(float(part[p])))
            want4[i, j] = acc
    got4 = oracle.gemm_int8_emulated(xq, xs, w_blob, m, n, k, ranges=4)
    assert np.array_equal(bits(got4), bits(want4))
    # the association matters at this size (else the check above would not tell them apart)
    assert not np.array_equal(bits(got4), bits(got))

    xf = (xb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wdq = np_dequant(QuantType.Q8_0, w_blob, n, k).astype(np.float64)
    y64 = oracle.gemm_f64(xb, w_blob, m, n, k)
    assert np.allclose(y64, xf @ wdq.T, rtol=1e-12, atol=1e-12)
    wbf = (_round_bf16(wdq.astype(np.float32)).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert np.allclose(oracle.gemm_f64(xb, w_blob, m, n, k, bf16_weights=True), xf @ wbf.T, rtol=1e-12, atol=1e-12)


def _f32_rne(fr: Fraction) -> np.float32:
    """The float32 nearest to the rational `fr`, ties to even (a correctly rounded fp32 op)."""
    if fr == 0:
        return np.float32(0.0)
    a = np.float32(float(fr))
    cands = [np.nextafter(a, np.float32(-np.inf)), a, np.nextafter(a, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr), int(np.float32(c).view(np.uint32)) & 1))
    return np.float32(best)


def _round_bf16(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


# ---- batched and GEMM references ---------------------------------------------------------

@pytest.mark.parametrize("qt", FORMATS, ids=lambda q: q.name)
def test_matmul_f64_rows_equal_matvec_f64_and_numpy(qt):
    """ref_matmul_f64 (the fp64 reference of every batched GEMV check) is quantMatvec per row
    of x (CpuBackend.java:708-725): row b equals ref_matvec_f64 of x[b] bit for bit, and the
    whole product equals numpy's fp64 product of the independently decoded matrix."""
    rows, batch = 37, 5  # odd rows and batch
    cols = 2 * qt.block_elements if qt.block_elements > 32 else 96
    blob = S.quant_blocks(qt, 31, rows, cols)
    xs = S.activations_f32(32, batch * cols).reshape(batch, cols)
    got = oracle.matmul_f64(qt.id, blob, rows, cols, xs)
    assert got.shape == (batch, rows)
    for b in range(batch):
        row = oracle.matvec_f64(qt.id, blob, rows, cols, xs[b])
        assert np.array_equal(got[b].view(np.uint64), row.view(np.uint64)), b
    want = xs.astype(np.float64) @ np_dequant(qt, blob, rows, cols).astype(np.float64).T
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    # a mistake a batched loop can make: rows of x swapped between outputs
    assert not np.allclose(got[::-1], want, rtol=1e-6)


@pytest.mark.parametrize("qt", [QuantType.Q4_0, QuantType.Q4_K, QuantType.Q6_K, QuantType.Q8_0], ids=lambda q: q.name)
def test_gemm_references_any_format_against_numpy(qt):
    """ref_gemm_f64 / ref_gemm_bf16w_f64 for every format of the prefill GEMM: numpy's fp64
    product of the independently decoded weights (and of those weights rounded to bf16,
    round-to-nearest-even, by a separate numpy rounding), within 1e-12; on Q8_0 they equal the
    Q8_0 entry points bit for bit."""
    m, n = 3, 11
    k = 512
    w_blob = S.quant_blocks(qt, 41, n, k)
    xb = S.activations_bf16(42, m * k).reshape(m, k)
    xf = (xb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wdq = np_dequant(qt, w_blob, n, k)
    y64 = oracle.gemm_f64(xb, w_blob, m, n, k, qtype=qt.id)
    want = xf @ wdq.astype(np.float64).T
    assert np.allclose(y64, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    wbf = (_round_bf16(wdq).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ybf = oracle.gemm_f64(xb, w_blob, m, n, k, bf16_weights=True, qtype=qt.id)
    wantbf = xf @ wbf.T
    assert np.allclose(ybf, wantbf, rtol=1e-12, atol=1e-12 * np.abs(wantbf).max())
    # the bf16 rounding of the weights is visible at this size (the two are not the same check)
    assert not np.allclose(ybf, y64, rtol=1e-9, atol=0)
    if qt == QuantType.Q8_0:
        assert np.array_equal(y64.view(np.uint64), oracle.gemm_q8_f64(xb, w_blob, m, n, k).view(np.uint64))
        assert np.array_equal(ybf.view(np.uint64), oracle.gemm_q8_f64(xb, w_blob, m, n, k, True).view(np.uint64))


def test_gemm_reference_rejects_misaligned_k():
    blob = S.quant_blocks(QuantType.Q4_K, 1, 2, 256)
    xb = S.activations_bf16(2, 2 * 288)
    with pytest.raises(ValueError):
        oracle.gemm_f64(xb, blob, 2, 2, 288, qtype=QuantType.Q4_K.id)

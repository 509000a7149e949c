"""GPU parity of the prefill GEMM over Q4_0, Q4_K and Q6_K weights (bf16 variant) against
the CPU oracle, through the C ABI.

Semantics: Y = X . W^T, each row of Y the quantMatvec of a row of X (QuantizedOps.java:27;
CpuBackend.java:708-725), W the ggml-decoded weights (Q4_0 also the reference's own
CpuQ4Gemm.java:17-24 gather). The kernel rounds every decoded fp32 weight to bf16 and
accumulates bf16 x bf16 products in fp32, so the bars are:
  - within 2e-5 * ||y||inf of the fp64 product of X and the bf16-rounded weights (only the
    fp32 accumulation order differs), and within 1e-2 (north star's bf16-activation bar) of
    the fp64 product of X and the exact weights;
  - one-hot rows of X return bf16 of a weight column bit for bit (one non-zero product), so
    the in-kernel dequantization is pinned exactly, element by element;
  - repeated calls agree bit for bit.
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import oracle
from jax4j_amd import DType, IllegalArgumentException, QuantType
from jax4j_amd import _native as N
from jax4j_amd import synthetic as S

pytestmark = pytest.mark.gpu

TOL_BF16X = 1e-2
TOL_ACCUM = 2e-5
KQ = [QuantType.Q4_0, QuantType.Q4_K, QuantType.Q6_K]

# (M, N, K): tails in M and N, one and several stages and superblocks, and each tile the
# dispatch picks: 64 x 64 (small grids), 128 x 64 (M = 512, N = 4096) and 128 x 128
# (M = 1024, N = 4096).
SHAPES = [(1, 1, 256), (5, 37, 512), (33, 100, 768), (64, 64, 1024), (65, 130, 256), (130, 257, 1280),
          (200, 96, 2304), (257, 300, 512), (512, 4096, 256), (1024, 4096, 256)]


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rel_err(y, ref):
    return float(np.abs(y.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def bf16_round(f: np.ndarray) -> np.ndarray:
    """fp32 -> nearest-even bf16, returned as fp32 (an independent numpy rounding)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def sample_rows(m):
    return sorted({0, 1, 15, 16, m // 2, m - 2, m - 1} & set(range(m)))


def upload_case(backend, qt, m, n, k, seed):
    w_blob = S.quant_blocks(qt, seed, n, k)
    xb = S.activations_bf16(seed + 1, m * k).reshape(m, k)
    w = backend.upload_quantized(w_blob, qt, (n, k))
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    return w_blob, xb, w, x


def check_rows(got, xb, w_blob, qt, m, n, k, rows=None):
    """The tight bar against the bf16-weight product; against the exact product, the bound the
    bf16 rounding of each weight guarantees (|bf16(w) - w| <= 2^-9 |w|, so per output at most
    2^-9 sum |w x|, doubled for slack) and, where the output is large enough for a norm to mean
    something, north star's 1e-2 * ||y||inf (a single short dot product can cancel below it)."""
    rows = list(range(m)) if rows is None else rows
    sub = np.ascontiguousarray(xb[rows])
    yb = oracle.gemm_f64(sub, w_blob, len(rows), n, k, bf16_weights=True, qtype=qt.id)
    y64 = oracle.gemm_f64(sub, w_blob, len(rows), n, k, qtype=qt.id)
    g = got[rows].astype(np.float64)
    assert rel_err(g, yb) <= TOL_ACCUM
    xf = np.abs((sub.astype(np.uint32) << 16).view(np.float32).astype(np.float64))
    wabs = np.abs(oracle.dequant_matrix(qt.id, w_blob, n, k).astype(np.float64))
    bound = 2.0**-8 * (xf @ wabs.T) + TOL_ACCUM * np.abs(y64).max()
    assert (np.abs(g - y64) <= bound).all()
    if len(rows) * n >= 4096:
        assert rel_err(g, y64) <= TOL_BF16X


@pytest.mark.parametrize("qt", KQ, ids=lambda q: q.name)
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_kquant_matches_oracle(backend, qt, m, n, k):
    note("gemm kquant", qt.name, m, n, k)
    w_blob, xb, w, x = upload_case(backend, qt, m, n, k, 7000 + m + n + k)
    y = backend.quant_matmul(w, x, "bf16")
    got = backend.download(y).reshape(m, n)
    check_rows(got, xb, w_blob, qt, m, n, k, sample_rows(m) if m * n * k > 2**26 else None)
    y2 = backend.quant_matmul(w, x, "bf16")
    assert np.array_equal(bits(backend.download(y2).reshape(m, n)), bits(got))
    for h in (w, x, y, y2):
        backend.release(h)


@pytest.mark.parametrize("qt,n,k", [(QuantType.Q4_K, 14336, 4096), (QuantType.Q6_K, 4096, 14336),
                                    (QuantType.Q4_0, 11008, 4096)], ids=lambda v: getattr(v, "name", str(v)))
@pytest.mark.parametrize("m", [32, 512])
def test_gemm_kquant_full_size(backend, qt, n, k, m):
    """configs[2]'s matrices (and configs[1]'s Q4_0 one) as prefill GEMMs at M = 32 and 512:
    sampled rows of X against the oracle."""
    note("gemm kquant full", qt.name, m, n, k)
    w_blob, xb, w, x = upload_case(backend, qt, m, n, k, 0x5EED9 + m)
    y = backend.quant_matmul(w, x, "bf16")
    got = backend.download(y).reshape(m, n)
    assert np.isfinite(got).all()
    check_rows(got, xb, w_blob, qt, m, n, k, [0, 1, m // 2, m - 1])
    for h in (w, x, y):
        backend.release(h)


@pytest.mark.parametrize("qt", KQ, ids=lambda q: q.name)
def test_gemm_kquant_one_hot_rows_return_bf16_weights(backend, qt):
    """Row r of X is the unit vector e_{k_r}: row r of Y is bf16 of weight column k_r, bit for
    bit. The k_r cover every element position of a 32-block, both superblock halves of a stage
    and several stages, so every lane group's unpack is checked against the oracle's decoder."""
    n, k = 96, 1024
    note("gemm kquant one-hot", qt.name, n, k)
    ks = sorted(set(list(range(0, 32)) + list(range(128, 160)) + [255, 256, 300, 511, 512, 777, 1000, 1023]))
    m = len(ks)
    w_blob = S.quant_blocks(qt, 91, n, k)
    xb = np.zeros((m, k), np.uint16)
    for r, kk in enumerate(ks):
        xb[r, kk] = 0x3F80  # bf16 1.0
    w = backend.upload_quantized(w_blob, qt, (n, k))
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    y = backend.quant_matmul(w, x, "bf16")
    got = backend.download(y).reshape(m, n)
    wd = oracle.dequant_matrix(qt.id, w_blob, n, k)
    want = bf16_round(wd[:, ks].T)
    # a decoded -0 (Q6_K: d sc (q - 32) with q = 32 and sc < 0) still sums to +0: the
    # accumulator starts at +0 and +0 + -0 = +0, so a GEMM output is never -0
    want = np.where(want == 0, np.float32(0.0), want)
    assert np.array_equal(bits(got), bits(want))
    for h in (w, x, y):
        backend.release(h)


# (70, 160, 512): one K range; (20, 96, 4096): 32-row tiles and K in 8 ranges; (45, 130,
# 2048): 64-row tiles, K in 4 ranges, and an output of M * N % 4 != 0 (the range sums take
# one element per thread)
@pytest.mark.parametrize("qt", KQ, ids=lambda q: q.name)
@pytest.mark.parametrize("m,n,k", [(70, 160, 512), (20, 96, 4096), (45, 130, 2048)])
def test_gemm_kquant_into_and_noalloc_match(backend, qt, m, n, k):
    """The three entry points agree bit for bit, also where K is split over workgroups (the
    partial products then go through stream-ordered memory, or the engine's fixed array in
    the allocation-free call, and are added in range order), and match the oracle."""
    note("gemm kquant into / noalloc", qt.name, m, n, k)
    w_blob, xb, w, x = upload_case(backend, qt, m, n, k, 88 + m)
    y_ref = backend.download(backend.quant_matmul(w, x, "bf16")).reshape(m, n)
    check_rows(y_ref, xb, w_blob, qt, m, n, k)
    lib = N.load()
    ptr = lambda h: backend.buffer_desc(h).device_ptr
    for fn in ("into", "noalloc"):
        yb = backend.upload(np.zeros((m, n), np.float32))
        if fn == "into":
            rc = lib.j4q_quant_matmul_into(w.handle, C.c_void_p(ptr(x)), m, N.GEMM_BF16, None, None, C.c_void_p(ptr(yb)), None)
        else:
            rc = lib.j4q_quant_matmul_noalloc(w.handle, C.c_void_p(ptr(x)), m, N.GEMM_BF16, C.c_void_p(ptr(yb)), None)
        assert rc == N.J4Q_OK, N.last_error()
        backend.sync()
        assert np.array_equal(bits(backend.download(yb).reshape(m, n)), bits(y_ref)), fn
        backend.release(yb)
    backend.release(w)
    backend.release(x)


def test_gemm_kquant_errors(backend):
    x = backend.upload(S.activations_bf16(4, 2 * 256).reshape(2, 256), shape=(2, 256), dtype=DType.BF16)
    wk = backend.upload_quantized(S.quant_blocks(QuantType.Q4_K, 3, 8, 256), QuantType.Q4_K, (8, 256))
    with pytest.raises(IllegalArgumentException, match="int8 variant needs Q8_0"):
        backend.quant_matmul(wk, x, "int8")
    w2 = backend.upload_quantized(S.quant_blocks(QuantType.Q2_0, 3, 8, 256), QuantType.Q2_0, (8, 256))
    with pytest.raises(IllegalArgumentException, match="no GEMM for type 42"):
        backend.quant_matmul(w2, x, "bf16")
    x96 = backend.upload(S.activations_bf16(5, 2 * 96).reshape(2, 96), shape=(2, 96), dtype=DType.BF16)
    w40 = backend.upload_quantized(S.quant_blocks(QuantType.Q4_0, 3, 8, 96), QuantType.Q4_0, (8, 96))
    with pytest.raises(IllegalArgumentException, match="no GEMM for type 2 with 96 columns"):
        backend.quant_matmul(w40, x96, "bf16")
    for h in (x, wk, w2, x96, w40):
        backend.release(h)

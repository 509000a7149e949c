"""GPU parity of the prefill GEMM (Q8_0 weights x bf16 activations) and the activation
quantizer against the CPU oracle, through the C ABI.

Bars: the quantizer is bit-exact; the int8 variant is bit-identical to the oracle's
emulation of the int8 arithmetic (exact int32 block dots folded in block order with one
fp32 FMA each) and within 1e-2 * ||y||inf of the exact product of the bf16 activations
and the exact dequantized weights; the bf16 variant is within 2e-5 * ||y||inf of the exact
product with bf16-rounded weights (only fp32 accumulation order differs) and within 1e-2
of the exact product.
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

TOL_BF16X = 1e-2  # bf16-activation configs
TOL_ACCUM = 2e-5  # fp32 accumulation-order difference only

# (M, N, K): tails in every dimension, one K block, the benchmark K, M above one tile. The
# bf16 variant runs M <= 32 and 33..192 on the small-M kernel (16 weight rows per workgroup,
# stages of 512 or 256 k: K = 32, 256 and 4096 cover a partial first stage, one stage and
# many) and 193..511 on the older 4-wave kernel when the grid is too small for the kernels
# that load their tiles straight into LDS (WIDE_SHAPES below cover those). The int8 variant runs N % 8 == 0 on the
# 2-wave 16 x 32 tile kernel up to M = 256 and the 8-wave 64 x 128 one above; N % 8 != 0
# (257 here) on the older 4-wave kernel.
SHAPES = [(1, 32, 32), (5, 13, 256), (33, 96, 512), (128, 128, 128), (130, 257, 1024), (64, 384, 4096),
          (32, 200, 4096), (100, 48, 800), (192, 96, 512), (200, 64, 256)]


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def int8_ranges(m, n, k):
    """K ranges of the int8 kernel the dispatch picks: four on the small-M kernel (M <= 256,
    N % 8 == 0) when it has at most 256 16 x 32 tiles, else one fold over all of K."""
    tiles = -(-m // 16) * -(-n // 32)
    return 4 if m <= 256 and n % 8 == 0 and n * k < 2**31 and tiles <= 256 else 1


def rel_err(y, ref):
    return float(np.abs(y.astype(np.float64) - ref).max() / max(np.abs(ref).max(), 1e-30))


def upload_case(backend, m, n, k, seed):
    w_blob = S.quant_blocks(QuantType.Q8_0, seed, n, k)
    xb = S.activations_bf16(seed + 1, m * k).reshape(m, k)
    w = backend.upload_quantized(w_blob, QuantType.Q8_0, (n, k))
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    return w_blob, xb, w, x


@pytest.mark.parametrize("m,k", [(1, 32), (5, 256), (128, 4096), (3, 14336)])
def test_quantize_act_bit_exact(backend, m, k):
    note("quantize_act", m, k)
    xb = S.activations_bf16(7 + m, m * k).reshape(m, k)
    xb[0, :32] = 0  # an all-zero block: scale 0, quants 0
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    qh, sh = backend.quantize_act(x)
    q = backend.download_raw(qh).reshape(m, k)
    s = backend.download(sh).reshape(m, k // 32)
    q_ref, s_ref = oracle.quantize_act(xb, m, k)
    assert np.array_equal(q, q_ref)
    assert np.array_equal(bits(s), bits(s_ref))
    for h in (x, qh, sh):
        backend.release(h)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_int8_matches_emulation_bit_exact(backend, m, n, k):
    note("gemm int8", m, n, k)
    w_blob, xb, w, x = upload_case(backend, m, n, k, 1000 + m + n + k)
    y = backend.quant_matmul(w, x, "int8")
    assert y.shape == (m, n)
    got = backend.download(y).reshape(m, n)
    xq, xs = oracle.quantize_act(xb, m, k)
    emu = oracle.gemm_int8_emulated(xq, xs, w_blob, m, n, k, ranges=int8_ranges(m, n, k))
    assert np.array_equal(bits(got), bits(emu))
    assert rel_err(got, oracle.gemm_f64(xb, w_blob, m, n, k)) <= TOL_BF16X
    for h in (w, x, y):
        backend.release(h)


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_bf16_matches_reference(backend, m, n, k):
    note("gemm bf16", m, n, k)
    w_blob, xb, w, x = upload_case(backend, m, n, k, 2000 + m + n + k)
    y = backend.quant_matmul(w, x, "bf16")
    got = backend.download(y).reshape(m, n)
    assert rel_err(got, oracle.gemm_f64(xb, w_blob, m, n, k, bf16_weights=True)) <= TOL_ACCUM
    assert rel_err(got, oracle.gemm_f64(xb, w_blob, m, n, k)) <= TOL_BF16X
    for h in (w, x, y):
        backend.release(h)


# The int8 kernels with N % 8 == 0 (stages of four blocks): one block; a partial last stage
# (K = 96, 160, 800); tails in M and N; the benchmark K; both sides of the M = 256 switch
# between the 16 x 32 and 64 x 128 tile kernels, and on the 16 x 32 kernel both sides of
# its 256-tile switch between four K ranges (K = 800, 2080, 4096: uneven ranges) and one
# ((96, 3000): 564 tiles). Every case is bit-identical to the emulation with the same
# association (blocks in order within each range, ranges added in order).
INT8_WIDE_SHAPES = [(65, 8, 32), (512, 136, 96), (600, 1024, 4096), (2048, 256, 160), (100, 48, 800),
                    (7, 40, 4096), (256, 64, 1024), (257, 64, 1024), (30, 1000, 2080), (96, 3000, 160)]


@pytest.mark.parametrize("m,n,k", INT8_WIDE_SHAPES)
def test_gemm_int8_wide_tiles_bit_exact(backend, m, n, k):
    note("gemm int8 wide", m, n, k)
    w_blob, xb, w, x = upload_case(backend, m, n, k, 4000 + m + n + k)
    y = backend.quant_matmul(w, x, "int8")
    got = backend.download(y).reshape(m, n)
    xq, xs = oracle.quantize_act(xb, m, k)
    assert np.array_equal(bits(got), bits(oracle.gemm_int8_emulated(xq, xs, w_blob, m, n, k, ranges=int8_ranges(m, n, k))))
    for h in (w, x, y):
        backend.release(h)


# The int8 kernels take the scale products fl(sx * dw) from an fp32 outer-product MFMA,
# a * b + 0 rounded once: bit-identical to the product except that a zero product comes out
# +0 where the product is -0 (sx = 0 against a negative dw, or dw = -0). The fold
# fma(float(I), p, acc) cannot tell them apart, since acc starts at +0 and never becomes -0.
# Planted here: all-zero activation blocks (sx = 0), weight blocks with d = +0, -0 and
# negative d, on the 16 x 32 kernel (four K ranges and one) and the 64 x 128 kernel.
@pytest.mark.parametrize("m,n,k", [(64, 64, 256), (96, 3000, 160), (512, 136, 256)])
def test_gemm_int8_zero_and_negative_scales_bit_exact(backend, m, n, k):
    note("gemm int8 zero scales", m, n, k)
    seed = 5000 + m + n + k
    w_blob = S.quant_blocks(QuantType.Q8_0, seed, n, k)
    nb = k // 32
    blocks = w_blob.reshape(n * nb, 34)
    d = blocks[:, :2].copy().view(np.uint16).reshape(-1)
    rng = np.random.default_rng(seed)
    pick = rng.permutation(n * nb)
    d[pick[0::7]] = 0x0000  # +0
    d[pick[1::7]] = 0x8000  # -0
    d[pick[2::7]] |= 0x8000  # negative
    blocks[:, :2] = d.view(np.uint8).reshape(-1, 2)
    xb = S.activations_bf16(seed + 1, m * k).reshape(m, k)
    for r in range(0, m, 3):
        b = (r * 5) % nb
        xb[r, 32 * b:32 * b + 32] = 0  # sx = 0
    w = backend.upload_quantized(w_blob, QuantType.Q8_0, (n, k))
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    y = backend.quant_matmul(w, x, "int8")
    got = backend.download(y).reshape(m, n)
    xq, xs = oracle.quantize_act(xb, m, k)
    assert (xs == 0).any() and (d == 0x8000).any()
    emu = oracle.gemm_int8_emulated(xq, xs, w_blob, m, n, k, ranges=int8_ranges(m, n, k))
    assert np.array_equal(bits(got), bits(emu))
    for h in (w, x, y):
        backend.release(h)


# M >= 512 runs the wide-tile kernel: 128 x 64 tiles while 128 x 128 ones would be fewer
# than 256 (one stage; a half stage at the end; tails in M and N), 128 x 128 from 256 tiles.
# The bf16 variant above M = 64 with even N loads its tiles straight into LDS when the grid
# is large enough: 128 x 128 tiles from 256 of them ((2048, 2048), (1030, 4098)), else
# 128 x 64 from 192 ((384, 4096)), else 64 x 64 from 128 ((96, 4096), (200, 2048)); smaller
# grids ((512, 128), (600, 200), (640, 520)) and odd N ((512, 129), (2048, 2049)) run the
# register-staged kernel at M >= 512. K = 64, 96 and 160 end in a partial stage.
WIDE_SHAPES = [(512, 128, 64), (600, 200, 96), (640, 520, 2048), (2048, 2048, 128), (1030, 4098, 160),
               (512, 129, 256), (2048, 2049, 64), (384, 4096, 128), (96, 4096, 160), (200, 2048, 96)]


@pytest.mark.parametrize("m,n,k", WIDE_SHAPES)
def test_gemm_bf16_wide_tiles(backend, m, n, k):
    note("gemm bf16 wide", m, n, k)
    w_blob, xb, w, x = upload_case(backend, m, n, k, 3000 + m + n + k)
    y = backend.quant_matmul(w, x, "bf16")
    got = backend.download(y).reshape(m, n)
    assert rel_err(got, oracle.gemm_f64(xb, w_blob, m, n, k, bf16_weights=True)) <= TOL_ACCUM
    assert rel_err(got, oracle.gemm_f64(xb, w_blob, m, n, k)) <= TOL_BF16X
    # repeated calls agree bit for bit
    for _ in range(3):
        y2 = backend.quant_matmul(w, x, "bf16")
        assert np.array_equal(bits(backend.download(y2).reshape(m, n)), bits(got))
        backend.release(y2)
    for h in (w, x, y):
        backend.release(h)


@pytest.mark.parametrize("m,n,k", [(512, 128, 256), (2048, 2048, 128)])
def test_gemm_bf16_lds_kernel_matches_register_staged(backend, m, n, k):
    """The two M >= 512 bf16 kernels give every block to the same wave in the same order, so
    the first n columns of an (n + 1)-row matrix (odd: register-staged kernel) equal the
    n-row matrix's (even: LDS-loading kernel) bit for bit."""
    note("gemm bf16 lds vs wide", m, n, k)
    w_blob = S.quant_blocks(QuantType.Q8_0, 5000 + m + n, n + 1, k)
    xb = S.activations_bf16(5001 + m, m * k).reshape(m, k)
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    w_odd = backend.upload_quantized(w_blob, QuantType.Q8_0, (n + 1, k))
    head = np.ascontiguousarray(np.frombuffer(bytes(w_blob), dtype=np.uint8)[: n * (k // 32) * 34])
    w_even = backend.upload_quantized(head, QuantType.Q8_0, (n, k))
    y_odd = backend.quant_matmul(w_odd, x, "bf16")
    y_even = backend.quant_matmul(w_even, x, "bf16")
    a = backend.download(y_odd).reshape(m, n + 1)[:, :n]
    b = backend.download(y_even).reshape(m, n)
    assert np.array_equal(bits(a), bits(b))
    for h in (x, w_odd, w_even, y_odd, y_even):
        backend.release(h)


@pytest.mark.parametrize("m", [32, 128, 512, 2048])
def test_gemm_full_size_rows_and_variants_agree(backend, m):
    """configs[3] at full size (N = K = 4096, every M of the sweep): sampled rows (first and
    last rows of the first, a middle and the last M tile) against the oracle, the int8 variant
    bit for bit against the emulation with the dispatch's K ranges, the bf16 variant within
    the accumulation-order bound of the bf16-weight product, and the two variants against each
    other over the whole output."""
    n, k = 4096, 4096
    note("gemm full", m, n, k)
    w_blob, xb, w, x = upload_case(backend, m, n, k, 0x5EED8 + m)
    yi = backend.quant_matmul(w, x, "int8")
    yb = backend.quant_matmul(w, x, "bf16")
    gi = backend.download(yi).reshape(m, n)
    gb = backend.download(yb).reshape(m, n)
    rows = sorted({0, 1, 15, 16, m // 2 - 1, m // 2, m - 17, m - 2, m - 1})
    sub = np.ascontiguousarray(xb[rows])
    y64 = oracle.gemm_f64(sub, w_blob, len(rows), n, k)
    assert rel_err(gi[rows], y64) <= TOL_BF16X
    assert rel_err(gb[rows], y64) <= TOL_BF16X
    xq, xs = oracle.quantize_act(sub, len(rows), k)
    emu = oracle.gemm_int8_emulated(xq, xs, w_blob, len(rows), n, k, ranges=int8_ranges(m, n, k))
    assert np.array_equal(bits(gi[rows]), bits(emu))
    assert rel_err(gb[rows], oracle.gemm_f64(sub, w_blob, len(rows), n, k, bf16_weights=True)) <= TOL_ACCUM
    assert rel_err(gi, gb.astype(np.float64)) <= 2 * TOL_BF16X
    for h in (w, x, yi, yb):
        backend.release(h)


@pytest.mark.parametrize("qt", [QuantType.Q8_0, QuantType.Q4_K], ids=lambda q: q.name)
def test_gemm_while_the_buffer_table_grows(backend, qt):
    """Regression: j4q_quant_matmul registers its output after looking up W and X, and that
    registration can move the engine's buffer table. The bf16 dispatch once read W's type
    through the stale pointer and failed with 'invalid argument' whenever the table grew on
    that call. Here 300 calls keep their outputs alive, so the table grows many times during
    a call; every call must succeed and equal the first bit for bit."""
    m, n, k = 96, 64, 256
    note("gemm while the table grows", qt.name)
    w_blob = S.quant_blocks(qt, 77, n, k)
    xb = S.activations_bf16(78, m * k).reshape(m, k)
    w = backend.upload_quantized(w_blob, qt, (n, k))
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    ys = [backend.quant_matmul(w, x, "bf16") for _ in range(300)]
    first = bits(backend.download(ys[0]).reshape(m, n))
    for y in (ys[1], ys[127], ys[128], ys[255], ys[256], ys[-1]):
        assert np.array_equal(bits(backend.download(y).reshape(m, n)), first)
    for h in ys + [w, x]:
        backend.release(h)


def test_gemm_into_caller_memory_matches(backend):
    """j4q_quant_matmul_into on engine-owned device memory gives the allocating call's result."""
    m, n, k = 70, 160, 512
    note("gemm into", m, n, k)
    w_blob, xb, w, x = upload_case(backend, m, n, k, 77)
    lib = N.load()
    for variant in ("int8", "bf16"):
        y_ref = backend.download(backend.quant_matmul(w, x, variant)).reshape(m, n)
        yb = backend.upload(np.zeros((m, n), np.float32))
        xq = backend.upload(np.zeros((m, k), np.float32))  # large enough for int8 [m, k]
        xs = backend.upload(np.zeros((m, k // 32), np.float32))
        ptr = lambda h: backend.buffer_desc(h).device_ptr
        v = N.GEMM_INT8 if variant == "int8" else N.GEMM_BF16
        rc = lib.j4q_quant_matmul_into(w.handle, C.c_void_p(ptr(x)), m, v, C.c_void_p(ptr(xq)), C.c_void_p(ptr(xs)), C.c_void_p(ptr(yb)), None)
        assert rc == N.J4Q_OK, N.last_error()
        backend.sync()
        assert np.array_equal(bits(backend.download(yb).reshape(m, n)), bits(y_ref))
        for h in (yb, xq, xs):
            backend.release(h)
    backend.release(w)
    backend.release(x)


@pytest.mark.parametrize("m,n1,n2,k", [(70, 160, 96, 512), (512, 4096, 1024, 4096)])
def test_gemm_prequantized_reuses_one_x(backend, m, n1, n2, k):
    """j4q_quant_matmul_q8_into on the activations j4q_quant_matmul_into's int8 variant left in
    its workspace for one matrix equals the int8 call on a second matrix bit for bit: one X,
    quantized once, feeding two Q8_0 matrices."""
    note("gemm prequantized", m, n1, n2, k)
    lib = N.load()
    ptr = lambda h: backend.buffer_desc(h).device_ptr
    xb = S.activations_bf16(91, m * k).reshape(m, k)
    x = backend.upload(xb, shape=(m, k), dtype=DType.BF16)
    w1 = backend.upload_quantized(S.quant_blocks(QuantType.Q8_0, 92, n1, k), QuantType.Q8_0, (n1, k))
    w2 = backend.upload_quantized(S.quant_blocks(QuantType.Q8_0, 93, n2, k), QuantType.Q8_0, (n2, k))
    xq = backend.upload(np.zeros((m, k // 4), np.float32))  # int8 [m, k]
    xs = backend.upload(np.zeros((m, k // 32), np.float32))
    y1 = backend.upload(np.zeros((m, n1), np.float32))
    y2 = backend.upload(np.zeros((m, n2), np.float32))
    rc = lib.j4q_quant_matmul_into(w1.handle, C.c_void_p(ptr(x)), m, N.GEMM_INT8, C.c_void_p(ptr(xq)),
                                   C.c_void_p(ptr(xs)), C.c_void_p(ptr(y1)), None)
    assert rc == N.J4Q_OK, N.last_error()
    rc = lib.j4q_quant_matmul_q8_into(w2.handle, C.c_void_p(ptr(xq)), C.c_void_p(ptr(xs)), m, C.c_void_p(ptr(y2)), None)
    assert rc == N.J4Q_OK, N.last_error()
    backend.sync()
    ref2 = backend.download(backend.quant_matmul(w2, x, "int8")).reshape(m, n2)
    assert np.array_equal(bits(backend.download(y2).reshape(m, n2)), bits(ref2))
    ref1 = backend.download(backend.quant_matmul(w1, x, "int8")).reshape(m, n1)
    assert np.array_equal(bits(backend.download(y1).reshape(m, n1)), bits(ref1))
    # the refusals: a Q4_0 matrix, NULL or misaligned pointers, m <= 0
    w4 = backend.upload_quantized(S.quant_blocks(QuantType.Q4_0, 94, 8, k), QuantType.Q4_0, (8, k))
    assert lib.j4q_quant_matmul_q8_into(w4.handle, C.c_void_p(ptr(xq)), C.c_void_p(ptr(xs)), m, C.c_void_p(ptr(y2)), None) == N.J4Q_EUNSUPPORTED
    assert lib.j4q_quant_matmul_q8_into(w2.handle, None, C.c_void_p(ptr(xs)), m, C.c_void_p(ptr(y2)), None) == N.J4Q_EINVAL
    assert lib.j4q_quant_matmul_q8_into(w2.handle, C.c_void_p(ptr(xq) + 4), C.c_void_p(ptr(xs)), m, C.c_void_p(ptr(y2)), None) == N.J4Q_EINVAL
    assert lib.j4q_quant_matmul_q8_into(w2.handle, C.c_void_p(ptr(xq)), C.c_void_p(ptr(xs)), 0, C.c_void_p(ptr(y2)), None) == N.J4Q_EINVAL
    for h in (x, w1, w2, w4, xq, xs, y1, y2):
        backend.release(h)


def test_gemm_errors(backend):
    w4 = backend.upload_quantized(S.quant_blocks(QuantType.Q4_0, 3, 8, 64), QuantType.Q4_0, (8, 64))
    x = backend.upload(S.activations_bf16(4, 2 * 64).reshape(2, 64), shape=(2, 64), dtype=DType.BF16)
    with pytest.raises(IllegalArgumentException, match="int8 variant needs Q8_0"):
        backend.quant_matmul(w4, x, "int8")
    w8 = backend.upload_quantized(S.quant_blocks(QuantType.Q8_0, 3, 8, 96), QuantType.Q8_0, (8, 96))
    with pytest.raises(IllegalArgumentException, match="shape mismatch"):
        backend.quant_matmul(w8, x, "bf16")
    with pytest.raises(IllegalArgumentException, match="variant"):
        backend.quant_matmul(w8, x, "fp8")
    for h in (w4, x, w8):
        backend.release(h)

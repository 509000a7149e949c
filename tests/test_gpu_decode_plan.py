"""The decode-step plan (j4q_decode_plan_*): a reduced decoder step against the eager
composition of quantMatvec / quantMatvecAdd calls and against the CPU oracle.

Per layer the plan computes qkv = [q|k|v].h, h' = o.x_o + h, gate_up = [gate|up].h',
h = down.x_down + h', then logits = head.h, replayed as one captured HIP graph
(QuantizedOps.java:27-30; CpuBackend.java:708-736 per GEMV). The plan runs the same kernels
as the single calls, so its outputs equal the eager composition bit for bit; against the
fp64 oracle chain the fp32 residual stream adds its roundings, bound 1e-4 * ||ref||_inf
(10x inside the 1e-3 decode tolerance).

A second, wider model gives every batched GEMV several column windows (K above 2048 columns
at 9-16 batch rows, above 4096 at 3-8, all four formats), whose sums meet in a second launch
on the plan's own workspace in the plan and on stream-ordered memory in the single calls:
the two agree bit for bit, on every replay (the workspace is reused by every GEMV of a step).
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
from jax4j_amd.backend import DecodePlan

pytestmark = pytest.mark.gpu

Q4K, Q6K, Q8, Q40 = QuantType.Q4_K, QuantType.Q6_K, QuantType.Q8_0, QuantType.Q4_0


class Dims:
    def __init__(self, d, qr, kvr, ffn, vocab):
        self.D, self.QR, self.KVR, self.FFN, self.VOCAB = d, qr, kvr, ffn, vocab
        self.shapes = dict(q=(qr, d), k=(kvr, d), v=(kvr, d), o=(d, qr), gate=(ffn, d), up=(ffn, d), down=(d, ffn))


SMALL = Dims(512, 512, 256, 1024, 1000)
# every batched GEMV over several column windows: K = 2560 (q|k|v, o, gate|up, head) and 4352
# (down) have 2 and 3 windows at 16 rows, down 2 at 3-8 rows
WIDE = Dims(2560, 2560, 512, 4352, 1000)
# layer 0: one type per group (q|k|v and gate|up fused into one launch each); layer 1: v and
# up of other types (runs launched separately, outputs copied into the fused layout)
TYPES = [
    dict(q=Q4K, k=Q4K, v=Q4K, o=Q4K, gate=Q4K, up=Q4K, down=Q6K),
    dict(q=Q4K, k=Q4K, v=Q6K, o=Q40, gate=Q4K, up=Q8, down=Q6K),
]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def rel_err(y, y_ref):
    return float(np.abs(y.astype(np.float64) - y_ref).max() / max(np.abs(y_ref).max(), 1e-30))


def ptr(backend, buf):
    return backend.buffer_desc(buf).device_ptr


def build_model(backend, dims, seed):
    """Two layers of weights and a head (host blobs kept for the oracle)."""
    layers, blobs = [], []
    for types in TYPES:
        lw, lb = {}, {}
        for name, qt in types.items():
            rows, cols = dims.shapes[name]
            blob = S.quant_blocks(qt, seed, rows, cols)
            seed += 1
            lb[name] = (qt, blob)
            lw[name] = backend.upload_quantized(blob, qt, (rows, cols))
        layers.append(lw)
        blobs.append(lb)
    hblob = S.quant_blocks(Q6K, seed, dims.VOCAB, dims.D)
    head = backend.upload_quantized(hblob, Q6K, (dims.VOCAB, dims.D))
    return layers, blobs, head, hblob


def release_model(backend, m):
    layers, _, head, _ = m
    for lw in layers:
        for w in lw.values():
            backend.release(w)
    backend.release(head)


@pytest.fixture(scope="module")
def model(backend):
    m = build_model(backend, SMALL, 0xD0C)
    yield m
    release_model(backend, m)


@pytest.fixture(scope="module")
def wide_model(backend):
    m = build_model(backend, WIDE, 0xD1C)
    yield m
    release_model(backend, m)


def make_io(backend, B, dims=SMALL):
    D, QR, FFN, VOCAB = dims.D, dims.QR, dims.FFN, dims.VOCAB
    h0 = S.activations_f32(71 + B, B * D).reshape(B, D)
    xo = S.activations_f32(72 + B, B * QR).reshape(B, QR)
    xd = S.activations_f32(73 + B, B * FFN).reshape(B, FFN)
    L = len(TYPES)
    bufs = dict(
        h=backend.upload(h0, shape=(B, D)),
        h0=backend.upload(h0, shape=(B, D)),
        x_o=backend.upload(xo, shape=(B, QR)),
        x_down=backend.upload(xd, shape=(B, FFN)),
        qkv=backend.upload(np.zeros(L * B * (QR + 2 * dims.KVR), np.float32)),
        gate_up=backend.upload(np.zeros(L * B * 2 * FFN, np.float32)),
        logits=backend.upload(np.zeros(B * VOCAB, np.float32)),
    )
    return h0, xo, xd, bufs


def read(backend, bufs, B, dims=SMALL):
    L = len(TYPES)
    return (
        backend.download(bufs["h"]).reshape(B, dims.D),
        backend.download(bufs["qkv"]).reshape(L, B, dims.QR + 2 * dims.KVR),
        backend.download(bufs["gate_up"]).reshape(L, B, 2 * dims.FFN),
        backend.download(bufs["logits"]).reshape(B, dims.VOCAB),
    )


def eager(backend, layers, head, h0, xo, xd):
    """The same step as single engine calls, one after another."""
    B = h0.shape[0]

    def up(a):
        return backend.upload(a, shape=a.shape) if B > 1 else backend.upload(a[0])

    def mv(w, x, add=None):
        xb = up(x)
        if add is None:
            y = backend.quant_matvec(w, xb)
        else:
            ab = up(add)
            y = backend.quant_matvec_add(w, xb, ab)
            backend.release(ab)
        out = backend.download(y).reshape(B, -1)
        backend.release(y)
        backend.release(xb)
        return out

    h = h0.copy()
    qkvs, gus = [], []
    for lw in layers:
        qkvs.append(np.concatenate([mv(lw[n], h) for n in ("q", "k", "v")], axis=1))
        h = mv(lw["o"], xo, h)
        gus.append(np.concatenate([mv(lw[n], h) for n in ("gate", "up")], axis=1))
        h = mv(lw["down"], xd, h)
    return h, np.stack(qkvs), np.stack(gus), mv(head, h)


def oracle_chain(blobs, hblob, h0, xo, xd, dims=SMALL):
    def mm(qb, x):
        qt, blob = qb
        rows, cols = blob_shape[id(blob)]
        return oracle.matmul_f64(qt.id, blob, rows, cols, x.astype(np.float32))

    blob_shape = {}
    for lb in blobs:
        for name, (qt, blob) in lb.items():
            blob_shape[id(blob)] = dims.shapes[name]
    blob_shape[id(hblob)] = (dims.VOCAB, dims.D)
    h = h0.astype(np.float64)
    qkvs, gus = [], []
    for lb in blobs:
        # the oracle takes fp32 activations; the residual is carried in fp64 between GEMVs
        qkvs.append(np.concatenate([mm(lb[n], h) for n in ("q", "k", "v")], axis=1))
        h = mm(lb["o"], xo) + h
        gus.append(np.concatenate([mm(lb[n], h) for n in ("gate", "up")], axis=1))
        h = mm(lb["down"], xd) + h
    return h, np.stack(qkvs), np.stack(gus), mm((Q6K, hblob), h)


def check_plan(backend, m, B, dims):
    layers, blobs, head, hblob = m
    D, QR, KVR, FFN, VOCAB = dims.D, dims.QR, dims.KVR, dims.FFN, dims.VOCAB
    h0, xo, xd, bufs = make_io(backend, B, dims)
    io = {k: ptr(backend, bufs[k]) for k in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")}
    plan = backend.decode_plan(layers, head, B, io)
    info = plan.info()
    assert info["graph"] == 1 and info["layers"] == 2 and info["batch"] == B
    assert (info["d_model"], info["qkv_rows"], info["ffn"], info["vocab"]) == (D, QR + 2 * KVR, FFN, VOCAB)
    # layer 0: q|k|v, o, gate|up, down = 4 GEMVs; layer 1: q|k, v, o, gate, up, down = 6; head 1
    assert info["gemvs_per_step"] == 11
    sh = dims.shapes
    total = sum(t.byte_size_for(sh[n][0] * sh[n][1]) for types in TYPES for n, t in types.items())
    assert info["weight_bytes"] == total + Q6K.byte_size_for(VOCAB * D)

    ref_eager = eager(backend, layers, head, h0, xo, xd)
    ref64 = oracle_chain(blobs, hblob, h0, xo, xd, dims)
    lib = N.load()
    first = None
    for replay in range(3):
        # reset the residual stream from its saved copy (a kernel, like the plan's own work)
        assert lib.j4q_copy(C.c_void_p(io["h"]), C.c_void_p(ptr(backend, bufs["h0"])), B * D * 4, None) == 0
        plan.run()
        backend.sync()
        got = read(backend, bufs, B, dims)
        for name, g, e, r in zip(("h", "qkv", "gate_up", "logits"), got, ref_eager, ref64):
            assert np.array_equal(bits(g), bits(e)), f"replay {replay}: {name} differs from the eager calls"
            assert rel_err(g.reshape(-1), r.reshape(-1)) <= 1e-4, f"replay {replay}: {name} vs oracle"
        if first is None:
            first = got
        else:
            for g, f in zip(got, first):
                assert np.array_equal(bits(g), bits(f)), f"replay {replay} differs from the first"
        # eager engine work between replays
        x = backend.upload(S.activations_f32(replay, D))
        y = backend.quant_matvec(layers[0]["q"], x)
        backend.download(y)
        backend.release(y)
        backend.release(x)
    plan.destroy()
    for b in bufs.values():
        backend.release(b)


@pytest.mark.parametrize("B", [1, 3, 16])
def test_decode_plan_matches_eager_and_oracle(backend, model, B):
    note("decode plan", "B", B)
    check_plan(backend, model, B, SMALL)


@pytest.mark.parametrize("B", [3, 8, 16, 19])
def test_decode_plan_column_windows(backend, wide_model, B):
    note("decode plan, several column windows", "B", B)
    check_plan(backend, wide_model, B, WIDE)


def test_decode_plan_keeps_its_launches_across_gemv_policies(backend, model):
    """A plan replays the launches it captured: one built on the matrix cores still equals the
    eager calls on the matrix cores after j4q_set_gemv_policy switched to the fp32 kernel, and
    one built under the fp32 policy equals the eager calls under it."""
    B = 3
    note("decode plan across GEMV policies", "B", B)
    layers, _, head, _ = model
    lib = N.load()
    h0, xo, xd, bufs = make_io(backend, B)
    io = {k: ptr(backend, bufs[k]) for k in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")}

    def replay(plan):
        assert lib.j4q_copy(C.c_void_p(io["h"]), C.c_void_p(ptr(backend, bufs["h0"])), B * SMALL.D * 4, None) == 0
        plan.run()
        backend.sync()
        return read(backend, bufs, B)

    prev = backend.set_gemv_policy("matrix_cores")
    plans = []
    try:
        plans.append(backend.decode_plan(layers, head, B, io))
        ref_mc = eager(backend, layers, head, h0, xo, xd)
        backend.set_gemv_policy("fp32")
        plans.append(backend.decode_plan(layers, head, B, io))
        ref_fp = eager(backend, layers, head, h0, xo, xd)
        for plan, ref, tag in ((plans[0], ref_mc, "matrix cores"), (plans[1], ref_fp, "fp32")):
            for name, g, e in zip(("h", "qkv", "gate_up", "logits"), replay(plan), ref):
                assert np.array_equal(bits(g), bits(e)), f"{tag} plan: {name} differs from its eager calls"
        # the fp32 policy's rows are the single-row calls
        sh, sq, sg, sl = eager(backend, layers, head, h0[:1], xo[:1], xd[:1])
        fh, fq, fg, fl = ref_fp
        assert np.array_equal(bits(fh[0]), bits(sh[0])) and np.array_equal(bits(fl[0]), bits(sl[0]))
        assert np.array_equal(bits(fq[:, 0]), bits(sq[:, 0])) and np.array_equal(bits(fg[:, 0]), bits(sg[:, 0]))
    finally:
        backend.set_gemv_policy(prev)
        for plan in plans:
            plan.destroy()
        for b in bufs.values():
            backend.release(b)


def test_decode_plan_errors(backend, model):
    layers, _, head, _ = model
    B = 1
    _, _, _, bufs = make_io(backend, B)
    io = {k: ptr(backend, bufs[k]) for k in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")}
    bad = [dict(layers[0]), dict(layers[1])]
    bad[1]["o"] = layers[1]["down"]  # [512, 1024]: o must have d_model rows and o_cols columns
    with pytest.raises(IllegalArgumentException, match="layer 1"):
        backend.decode_plan(bad, head, B, io)
    with pytest.raises(IllegalArgumentException, match="NULL"):
        backend.decode_plan(layers, head, B, {**io, "x_o": 0})
    with pytest.raises(IllegalArgumentException, match="aligned"):
        backend.decode_plan(layers, head, B, {**io, "h": io["h"] + 4})
    plan = backend.decode_plan(layers, None, B, io)
    assert plan.info()["vocab"] == 0 and plan.info()["gemvs_per_step"] == 10
    stale = DecodePlan(backend, plan.handle)
    plan.destroy()
    with pytest.raises(IllegalArgumentException, match="unknown or destroyed"):
        stale.run()
    for b in bufs.values():
        backend.release(b)


def test_decode_plan_pins_the_matrices_it_reads(backend):
    """A plan's graph reads o, down, the head and every q/k/v or gate/up part it did not copy
    into a fused plan-owned matrix: releasing one of those while the plan lives is refused
    (the memory of a queued replay is never freed), the refused buffer stays valid, replays
    still equal the eager calls, and after j4q_decode_plan_destroy they release normally.
    Parts that were concatenated into plan-owned copies are not read by the graph and may be
    released at once. A GEMV trace set while the plan is created is not recorded in its
    graph: a replay after the trace was turned off writes nothing into the trace buffer."""
    note("decode plan pins")
    m = build_model(backend, SMALL, 0xD2C)
    layers, blobs, head, hblob = m
    B = 1
    h0, xo, xd, bufs = make_io(backend, B)
    io = {k: ptr(backend, bufs[k]) for k in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")}
    lib = N.load()
    sentinel = np.full(4 * 4096, 0x7FC00001, np.uint32).view(np.float32)  # a NaN pattern
    tr = backend.upload(sentinel)
    assert lib.j4q_gemv_trace(C.c_void_p(ptr(backend, tr)), sentinel.size // 2) == 0
    try:
        plan = backend.decode_plan(layers, head, B, io)
    finally:
        assert lib.j4q_gemv_trace(None, 0) == 0
    read_by_graph = [layers[0]["o"], layers[0]["down"], layers[1]["v"], layers[1]["o"], layers[1]["gate"],
                     layers[1]["up"], layers[1]["down"], head]
    for w in read_by_graph:
        with pytest.raises(IllegalArgumentException, match="live decode plan"):
            backend.release(w)
        assert w.handle != 0
    # layer 0's q, k, v (one type) and gate, up (one type) run from plan-owned concatenations
    fused_parts = [layers[0][n] for n in ("q", "k", "v", "gate", "up")] + [layers[1][n] for n in ("q", "k")]
    ref_eager = eager(backend, layers, head, h0, xo, xd)
    for w in fused_parts:
        backend.release(w)
    for replay in range(2):
        assert lib.j4q_copy(C.c_void_p(io["h"]), C.c_void_p(ptr(backend, bufs["h0"])), B * SMALL.D * 4, None) == 0
        plan.run()
        backend.sync()
        got = read(backend, bufs, B)
        for name, g, e in zip(("h", "qkv", "gate_up", "logits"), got, ref_eager):
            assert np.array_equal(bits(g), bits(e)), f"replay {replay}: {name} differs from the eager calls"
    assert np.array_equal(backend.download(tr).view(np.uint32), sentinel.view(np.uint32))
    plan.destroy()
    for w in read_by_graph:
        backend.release(w)
    for b in list(bufs.values()) + [tr]:
        backend.release(b)

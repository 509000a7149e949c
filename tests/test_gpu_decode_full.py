"""configs[4] at full size through the decode plan: 32 Llama-3-8B-shaped layers (q 4096x4096,
k/v 1024x4096, o 4096x4096, gate/up 14336x4096 in Q4_K; down 4096x14336 in Q6_K) and the
128256x4096 Q6_K output head, 4.84 GB of weights generated in HBM with the benchmark's
device generator, at batch 1 and 16 -- the step bench.py times.

One replay of the plan (fused q|k|v and gate|up, residual adds out of place between two
buffers, one captured HIP graph; at B = 16 the head's four column windows meet on the
plan-owned workspace) must equal the 225 eager stream-ordered calls bit for bit: every
per-layer output, the residual stream after the last layer and the logits. The eager calls
are checked against the CPU oracle at these exact shapes in test_gpu_decode_shapes.py
(QuantizedOps.java:27-30; CpuBackend.java:708-736 per GEMV).
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

from jax4j_amd import QuantType
from jax4j_amd import _native as N
from jax4j_amd import synthetic as S

pytestmark = pytest.mark.gpu

Q4K, Q6K = QuantType.Q4_K, QuantType.Q6_K
D, QR, KVR, FFN, VOCAB, LAYERS = 4096, 4096, 1024, 14336, 128256, 32
LAYER = [("q", Q4K, QR, D), ("k", Q4K, KVR, D), ("v", Q4K, KVR, D), ("o", Q4K, D, QR),
         ("gate", Q4K, FFN, D), ("up", Q4K, FFN, D), ("down", Q6K, D, FFN)]
WEIGHT_BYTES = 4841250816


def note(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def ptr(backend, buf):
    return backend.buffer_desc(buf).device_ptr


@pytest.fixture(scope="module")
def full_model(backend):
    """The 32 layers and the head, generated on the device (bench.py's seeds and generator)."""
    lib = N.load()
    note("full decode model: generating 4.84 GB of weights in HBM")
    stage_bytes = Q6K.byte_size_for(VOCAB * D)
    staging = backend.upload(np.zeros(stage_bytes // 4, np.float32))
    sp = ptr(backend, staging)
    seed = 0xDEC0DE

    def make(qt, rows, cols):
        nonlocal seed
        nbytes = qt.byte_size_for(rows * cols)
        assert nbytes <= stage_bytes
        rc = lib.j4q_synth_quant_device(qt.id, seed, rows, cols, C.c_void_p(sp), nbytes, None)
        assert rc == N.J4Q_OK, N.last_error()
        seed += 1
        return backend.upload_quantized_device(sp, nbytes, qt, (rows, cols))

    layers = []
    for _ in range(LAYERS):
        layers.append({name: make(qt, rows, cols) for name, qt, rows, cols in LAYER})
    head = make(Q6K, VOCAB, D)
    backend.release(staging)
    yield layers, head
    for lw in layers:
        for w in lw.values():
            backend.release(w)
    backend.release(head)


@pytest.mark.parametrize("B", [1, 16])
def test_full_decode_plan_equals_eager_calls(backend, full_model, B):
    layers, head = full_model
    note("full decode plan vs eager", "B", B)
    h0 = S.activations_f32(0xA11 + B, B * D).reshape(B, D)
    up = lambda a: backend.upload(np.ascontiguousarray(a, np.float32).reshape(-1))
    bufs = {
        "h": up(h0), "h0": up(h0),
        "x_o": up(S.activations_f32(0xA12 + B, B * QR)),
        "x_down": up(S.activations_f32(0xA13 + B, B * FFN)),
        "qkv": up(np.zeros(LAYERS * B * (QR + 2 * KVR))),
        "gate_up": up(np.zeros(LAYERS * B * 2 * FFN)),
        "logits": up(np.zeros(B * VOCAB)),
    }
    io = {k: ptr(backend, bufs[k]) for k in ("h", "x_o", "x_down", "qkv", "gate_up", "logits")}
    plan = backend.decode_plan(layers, head, B, io)
    info = plan.info()
    assert info["weight_bytes"] == WEIGHT_BYTES and info["gemvs_per_step"] == 4 * LAYERS + 1
    plan.run()
    backend.sync()
    p_h = backend.download(bufs["h"]).reshape(B, D)
    p_qkv = backend.download(bufs["qkv"]).reshape(LAYERS, B, QR + 2 * KVR)
    p_gu = backend.download(bufs["gate_up"]).reshape(LAYERS, B, 2 * FFN)
    p_logits = backend.download(bufs["logits"]).reshape(B, VOCAB)
    plan.destroy()

    # the same step as 225 stream-ordered calls on their own buffers
    e = {
        "h": up(h0), "ha": up(np.zeros(B * D)),
        "q": up(np.zeros(B * QR)), "k": up(np.zeros(B * KVR)), "v": up(np.zeros(B * KVR)),
        "gate": up(np.zeros(B * FFN)), "up": up(np.zeros(B * FFN)), "logits": up(np.zeros(B * VOCAB)),
    }
    ep = {k: ptr(backend, v) for k, v in e.items()}
    for l, lw in enumerate(layers):
        for n in ("q", "k", "v"):
            backend.quant_matvec_into(lw[n], ep["h"], 0, ep[n], B)
        backend.quant_matvec_into(lw["o"], io["x_o"], ep["h"], ep["ha"], B)
        for n in ("gate", "up"):
            backend.quant_matvec_into(lw[n], ep["ha"], 0, ep[n], B)
        backend.quant_matvec_into(lw["down"], io["x_down"], ep["ha"], ep["h"], B)
        qkv = np.concatenate([backend.download(e[n]).reshape(B, -1) for n in ("q", "k", "v")], axis=1)
        gu = np.concatenate([backend.download(e[n]).reshape(B, -1) for n in ("gate", "up")], axis=1)
        assert np.array_equal(bits(p_qkv[l]), bits(qkv)), f"layer {l} q|k|v"
        assert np.array_equal(bits(p_gu[l]), bits(gu)), f"layer {l} gate|up"
    backend.quant_matvec_into(head, ep["h"], 0, ep["logits"], B)
    assert np.array_equal(bits(p_h), bits(backend.download(e["h"]).reshape(B, D))), "residual stream"
    assert np.array_equal(bits(p_logits), bits(backend.download(e["logits"]).reshape(B, VOCAB))), "logits"
    assert np.isfinite(p_logits).all() and np.abs(p_logits).max() > 0
    for b in list(bufs.values()) + list(e.values()):
        backend.release(b)

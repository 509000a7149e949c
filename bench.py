#!/usr/bin/env python3
"""Benchmark of the MI355X GGUF quantized-matmul engine (one GPU).

The headline (`value`) is the benchmark's configs[4]: the Llama-3-8B-shaped decode step,
matmuls only, Q4_K_M mix (32 layers of q/k/v/o/gate/up Q4_K and down Q6_K, plus the 128256 x
4096 Q6_K output head: 4,841,250,816 bytes of weights), at batch 1, run through the engine's
decode-step plan (j4q_decode_plan_*: q|k|v and gate|up fused, both residual adds per layer
as quantMatvecAdd, one captured HIP graph per step). `value` is weight bytes streamed per
second; tokens/s = batch / step time. A "step" is one decode step.

The other configs are reported in `workloads`: configs[0] Q8_0 GEMV, configs[1] Q4_0 GEMV at
batch 1 and 8, configs[2] Q4_K / Q6_K GEMVs, configs[3] the Q8_0 prefill GEMM (int8 and bf16
variants, M = 32..2048), configs[4] at batch 16 and unfused without a graph.

Measurement: inputs are resident in HBM before timing. Each single-matrix workload rotates
over >= 512 MB of distinct weight copies so the 256 MB Infinity Cache cannot serve them (the
decode step streams 4.84 GB and needs no rotation). A bounded spin kernel holds the engine
stream while the host queues the timed launches, so they execute back to back; HIP events on
that same stream bracket exactly the K timed launches, with events between samples (15
samples, the method of GpuComparison.java:216-224,249-254), giving the mean over the region
and the median / min / p90 of the samples.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from jax4j_amd import QuantType  # noqa: E402
from jax4j_amd import _native as N  # noqa: E402
from jax4j_amd.backend import Mi355xBackend, check  # noqa: E402

METRIC = "quant GEMV HBM GB/s (% of peak) + prefill GEMM TOPS (% MFMA peak), 1 GPU"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5033.0
BF16_PEAK_TFLOPS = 2517.0
ROTATE_BYTES = 512 << 20
SAMPLES = 15
Q4K, Q6K = QuantType.Q4_K, QuantType.Q6_K
# per layer (name, type, rows, cols), then the output head
LLAMA3_8B_LAYER = [("q", Q4K, 4096, 4096), ("k", Q4K, 1024, 4096), ("v", Q4K, 1024, 4096), ("o", Q4K, 4096, 4096),
                   ("gate", Q4K, 14336, 4096), ("up", Q4K, 14336, 4096), ("down", Q6K, 4096, 14336)]
LLAMA3_8B_HEAD = (Q6K, 128256, 4096)
# The decode step's dominant kernel (the largest share of the step's time): the fused gate|up
# GEMV, 28672 x 4096 Q4_K at batch 1. Its HBM bytes per launch were measured with rocprofv3
# FETCH_SIZE / WRITE_SIZE counters scaled by a copy kernel of known size (see the .md beside it).
DOMINANT = "q4_k_gemv_gate_up_fused_b1"
# the decode step's four batch-1 GEMV shapes (name, type, rows, cols, concatenated parts)
STEP_SHAPES_B1 = (
    (DOMINANT, Q4K, 28672, 4096, [14336, 14336]),
    ("q4_k_gemv_qkv_fused_b1", Q4K, 6144, 4096, [4096, 1024, 1024]),
    ("q4_k_gemv_o_b1", Q4K, 4096, 4096, None),
    ("q6_k_gemv_down_b1", Q6K, 4096, 14336, None),
)
# hipDeviceAttribute_t value of hipDeviceAttributeWallClockRate (kHz of the clock j4q_gemv_trace stamps)
HIP_ATTR_WALL_CLOCK_RATE = 10017


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Hip:
    """The HIP runtime the engine library linked (same process-wide instance)."""

    def __init__(self):
        N.load()
        self.h = C.CDLL("libamdhip64.so.7")
        for name, args in {
            "hipMalloc": [C.POINTER(C.c_void_p), C.c_size_t],
            "hipFree": [C.c_void_p],
            "hipDeviceSynchronize": [],
            "hipEventCreate": [C.POINTER(C.c_void_p)],
            "hipEventDestroy": [C.c_void_p],
            "hipEventRecord": [C.c_void_p, C.c_void_p],
            "hipEventSynchronize": [C.c_void_p],
            "hipEventElapsedTime": [C.POINTER(C.c_float), C.c_void_p, C.c_void_p],
            "hipMemset": [C.c_void_p, C.c_int, C.c_size_t],
            "hipMemcpy": [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int],
            "hipDeviceGetAttribute": [C.POINTER(C.c_int), C.c_int, C.c_int],
        }.items():
            fn = getattr(self.h, name)
            fn.argtypes = args
            fn.restype = C.c_int

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with HIP error {rc}")

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self.ok(self.h.hipMalloc(C.byref(p), max(nbytes, 256)), "hipMalloc")
        return p.value

    def free(self, p: int) -> None:
        self.ok(self.h.hipFree(C.c_void_p(p)), "hipFree")

    def sync(self) -> None:
        self.ok(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def event(self) -> int:
        e = C.c_void_p()
        self.ok(self.h.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def event_free(self, e: int) -> None:
        self.ok(self.h.hipEventDestroy(C.c_void_p(e)), "hipEventDestroy")

    def record(self, e: int, stream: int) -> None:
        self.ok(self.h.hipEventRecord(C.c_void_p(e), C.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a: int, b: int) -> float:
        self.ok(self.h.hipEventSynchronize(C.c_void_p(b)), "hipEventSynchronize")
        ms = C.c_float()
        self.ok(self.h.hipEventElapsedTime(C.byref(ms), C.c_void_p(a), C.c_void_p(b)), "hipEventElapsedTime")
        return float(ms.value)


def stats_us(sample_ms, sample_launches):
    """median / min / p90 of the per-launch time (us) over samples."""
    per = sorted(1e3 * ms / n for ms, n in zip(sample_ms, sample_launches))
    k = len(per)
    med = per[k // 2] if k % 2 else 0.5 * (per[k // 2 - 1] + per[k // 2])
    p90 = per[min(k - 1, math.ceil(0.9 * k) - 1)]
    return {"median_us": round(med, 3), "min_us": round(per[0], 3), "p90_us": round(p90, 3), "samples": k}


class Engine:
    def __init__(self):
        self.be = Mi355xBackend()
        if not self.be.is_available():
            raise SystemExit("bench.py: no MI355X (gfx950) device is available")
        self.lib = self.be._lib()
        self.hip = Hip()
        self.stream = self.be.stream()
        self.info = self.be.device_info()

    def weights(self, qt: QuantType, rows: int, cols: int, seed: int):
        """A quantized matrix generated in HBM and uploaded through the device path."""
        nbytes = qt.byte_size_for(rows * cols)
        raw = self.hip.malloc(nbytes)
        check(self.lib.j4q_synth_quant_device(qt.id, seed, rows, cols, C.c_void_p(raw), nbytes, None), "synth")
        w = self.be.upload_quantized_device(raw, nbytes, qt, (rows, cols))
        self.hip.free(raw)
        return w, nbytes

    def f32(self, n: int, seed: int) -> int:
        p = self.hip.malloc(4 * n)
        check(self.lib.j4q_synth_f32_device(seed, n, C.c_void_p(p), None), "synth")
        return p

    def bf16(self, n: int, seed: int) -> int:
        p = self.hip.malloc(2 * n)
        check(self.lib.j4q_synth_bf16_device(seed, n, C.c_void_p(p), None), "synth")
        return p

    def time_region(self, enqueue, launches: int, host_us_per_launch: float = 30.0, samples: int = 1):
        """Queue `launches` launches (enqueue(i)) behind a spin kernel long enough for the host
        to queue them all, with HIP events on the engine stream at the region's ends and
        between `samples` equal samples. Returns the region's GPU time (ms), the samples' times
        and launch counts, the host's queueing time per launch (us), and whether the host was
        slower than the spin (then the GPU may have idled and the region is host-bound)."""
        self.hip.sync()
        samples = max(1, min(samples, launches))
        bounds = [round(i * launches / samples) for i in range(samples + 1)]
        evs = [self.hip.event() for _ in range(samples + 1)]
        spin_us = int(min(5_000_000, 3000 + 1.5 * launches * host_us_per_launch))
        check(self.lib.j4q_spin(spin_us, C.c_void_p(self.stream)), "spin")
        t0 = time.perf_counter()
        for k in range(samples):
            self.hip.record(evs[k], self.stream)
            for i in range(bounds[k], bounds[k + 1]):
                enqueue(i)
        self.hip.record(evs[samples], self.stream)
        host_us = (time.perf_counter() - t0) * 1e6
        total = self.hip.elapsed_ms(evs[0], evs[samples])
        sample_ms = [self.hip.elapsed_ms(evs[k], evs[k + 1]) for k in range(samples)]
        self.hip.sync()
        for e in evs:
            self.hip.event_free(e)
        if host_us > spin_us:
            log(f"warning: host queueing ({host_us:.0f} us) outlasted the spin ({spin_us} us); region may be host-bound")
        counts = [bounds[k + 1] - bounds[k] for k in range(samples)]
        return total, sample_ms, counts, host_us / max(launches, 1), host_us > spin_us


def gemv_workload(eng: Engine, name: str, qt: QuantType, rows: int, cols: int, batch: int, steps: int, warmup: int,
                  parts=None, rotate_bytes: int = ROTATE_BYTES):
    """GEMV launches over rotating weight copies. `parts` (row counts) builds each copy as a
    row concatenation (j4q_concat_rows), as the decode step fuses gate|up. us_per_launch comes
    from one region of `steps` back-to-back launches with events only at its ends (the
    rocprofv3 kernel average agrees with it); median / min / p90 come from a second region
    split into SAMPLES parts, whose inner events each add a small gap to the stream.
    rotate_bytes = 1 keeps one copy, which then stays in the Infinity Cache between launches."""
    blob_bytes = qt.byte_size_for(rows * cols)
    copies = max(1, math.ceil(rotate_bytes / blob_bytes))
    log(f"{name}: {qt.name} N={rows} K={cols} B={batch}, {copies} weight copies")
    ws = []
    for i in range(copies):
        if parts:
            ps = [eng.weights(qt, r, cols, 0x5EED5 + 97 * i + j)[0] for j, r in enumerate(parts)]
            ws.append(eng.be.concat_rows(ps))
            for p in ps:
                eng.be.release(p)
        else:
            ws.append(eng.weights(qt, rows, cols, 0x5EED5 + 97 * i)[0])
    x = eng.f32(batch * cols, 0x5EED6)
    y = eng.hip.malloc(4 * batch * rows)
    handles = [w.handle for w in ws]
    fn = eng.lib.j4q_quant_matvec_into
    s = C.c_void_p(eng.stream)
    xp, yp = C.c_void_p(x), C.c_void_p(y)

    def enqueue(i):
        rc = fn(handles[i % copies], xp, None, yp, batch, s)
        if rc:
            check(rc, name)

    _, _, _, host_us, _ = eng.time_region(enqueue, warmup)
    ms, _, _, _, host_bound = eng.time_region(enqueue, steps, host_us)
    per = ms / steps
    _, sms, cnt, _, _ = eng.time_region(enqueue, steps, host_us, SAMPLES)
    alg = blob_bytes + 4 * batch * cols + 4 * batch * rows
    gbs = alg / (per * 1e-3) / 1e9
    for w in ws:
        eng.be.release(w)
    eng.hip.free(x)
    eng.hip.free(y)
    st = stats_us(sms, cnt)
    log(f"{name}: {per * 1e3:.2f} us/launch (sampled: median {st['median_us']}, min {st['min_us']}, p90 {st['p90_us']}), "
        f"{gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
    return {
        "workload": name,
        "quant": qt.name,
        "N": rows,
        "K": cols,
        "batch": batch,
        "weight_copies": copies,
        "us_per_launch": round(per * 1e3, 3),
        "sampled": st,
        "algorithmic_bytes": alg,
        "GBps": round(gbs, 1),
        "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "host_bound": host_bound,
    }


class DecodeModel:
    """configs[4]'s weights (32 layers + head, generated in HBM once) and the step's
    activation buffers; plans are built from them per batch size."""

    def __init__(self, eng: Engine, layers: int = 32):
        self.eng = eng
        self.layers, self.total = [], 0
        seed = 0xDEC0DE
        for _ in range(layers):
            lw = {}
            for name, qt, n, k in LLAMA3_8B_LAYER:
                lw[name], nb = eng.weights(qt, n, k, seed)
                seed += 1
                self.total += nb
            self.layers.append(lw)
        self.head, nb = eng.weights(*LLAMA3_8B_HEAD, seed)
        self.total += nb

    def release(self):
        for lw in self.layers:
            for w in lw.values():
                self.eng.be.release(w)
        self.eng.be.release(self.head)


def decode_workload(eng: Engine, model: DecodeModel, batch: int, steps: int, warmup: int, plan: bool = True):
    """configs[4] at `batch`: with `plan`, one graph replay of the engine's decode plan per step
    (129 GEMV launches: q|k|v and gate|up fused); otherwise the 225 GEMVs as single
    stream-ordered calls (the residual adds out of place), for comparison."""
    L = len(model.layers)
    d, qkv_rows, ffn, vocab = 4096, 6144, 14336, LLAMA3_8B_HEAD[1]
    bufs = {
        "h": eng.f32(batch * d, 0xA11),
        "x_o": eng.f32(batch * d, 0xA12),
        "x_down": eng.f32(batch * ffn, 0xA13),
        "qkv": eng.hip.malloc(4 * L * batch * qkv_rows),
        "gate_up": eng.hip.malloc(4 * L * batch * 2 * ffn),
        "logits": eng.hip.malloc(4 * batch * vocab),
    }
    h2 = eng.hip.malloc(4 * batch * d)
    s = C.c_void_p(eng.stream)
    if plan:
        p = eng.be.decode_plan(model.layers, model.head, batch, bufs)
        info = p.info()
        assert info["weight_bytes"] == model.total, (info["weight_bytes"], model.total)
        launches = info["gemvs_per_step"]

        def enqueue(step):
            p.run(eng.stream)
    else:
        fn = eng.lib.j4q_quant_matvec_into
        calls = []
        h, ha = bufs["h"], h2
        for l, lw in enumerate(model.layers):
            q0 = bufs["qkv"] + 4 * l * batch * qkv_rows
            g0 = bufs["gate_up"] + 4 * l * batch * 2 * ffn
            # single calls write their own [batch, rows] outputs (at batch 1 the same layout)
            calls += [(lw["q"], h, 0, q0), (lw["k"], h, 0, q0 + 4 * batch * 4096), (lw["v"], h, 0, q0 + 4 * batch * 5120)]
            calls.append((lw["o"], bufs["x_o"], h, ha))
            calls += [(lw["gate"], ha, 0, g0), (lw["up"], ha, 0, g0 + 4 * batch * ffn)]
            calls.append((lw["down"], bufs["x_down"], ha, h))
        calls.append((model.head, h, 0, bufs["logits"]))
        calls = [(w.handle, C.c_void_p(x), C.c_void_p(a or None), C.c_void_p(y)) for w, x, a, y in calls]
        launches = len(calls)

        def enqueue(step):
            for wh, xp, ap, yp in calls:
                rc = fn(wh, xp, ap, yp, batch, s)
                if rc:
                    check(rc, "decode")

    _, _, _, host_us, _ = eng.time_region(enqueue, warmup, 30.0 * launches)
    ms, sms, cnt, _, host_bound = eng.time_region(enqueue, steps, host_us, SAMPLES)
    per = ms / steps
    if plan:
        p.destroy()
    for v in list(bufs.values()) + [h2]:
        eng.hip.free(v)
    gbs = model.total / (per * 1e-3) / 1e9
    st = stats_us(sms, cnt)
    tag = "plan (fused + graph)" if plan else "single calls"
    log(f"decode B={batch} {tag}: {per:.3f} ms/step (median {st['median_us'] / 1e3:.3f}), {gbs:.0f} GB/s weights, "
        f"{batch / (per * 1e-3):.0f} tok/s")
    return {
        "workload": f"llama3-8b decode step B={batch} {tag}",
        "gemvs_per_step": launches,
        "batch": batch,
        "ms_per_step": round(per, 4),
        **{k.replace("_us", "_ms"): (round(v / 1e3, 4) if k.endswith("_us") else v) for k, v in st.items()},
        "weight_bytes_per_step": model.total,
        "GBps": round(gbs, 1),
        "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(batch / (per * 1e-3), 1),
        "host_bound": host_bound,
    }


def gemm_workload(eng: Engine, m: int, variant: str, steps: int, warmup: int, n: int = 4096, k: int = 4096,
                  qt: QuantType = QuantType.Q8_0):
    """Q8_0 prefill GEMM Y[m, n] = X[m, k] . W^T with bf16 X; the int8 variant's
    timed call includes quantizing X (j4q_quant_matmul_into runs both kernels). Variant
    "int8q": the int8 GEMM alone on X quantized once before the region (j4q_quant_matmul_q8_into,
    as for one X feeding several matrices); not a configs[3] line. With another `qt` (Q4_0,
    Q4_K, Q6_K; bf16 variant) the same GEMM over configs[1]/[2]'s matrices."""
    blob_bytes = qt.byte_size_for(n * k)
    copies = max(1, math.ceil(ROTATE_BYTES / blob_bytes))
    ws = [eng.weights(qt, n, k, 0x5EED8 + 31 * i)[0] for i in range(copies)]
    x = eng.bf16(m * k, 0x5EED9)
    xq = eng.hip.malloc(m * k)
    xs = eng.hip.malloc(4 * m * (k // 32))
    y = eng.hip.malloc(4 * m * n)
    handles = [w.handle for w in ws]
    fn = eng.lib.j4q_quant_matmul_into
    v = N.GEMM_BF16 if variant == "bf16" else N.GEMM_INT8
    s = C.c_void_p(eng.stream)
    xp, xqp, xsp, yp = C.c_void_p(x), C.c_void_p(xq), C.c_void_p(xs), C.c_void_p(y)
    if variant == "int8q":
        check(fn(handles[0], xp, m, v, xqp, xsp, yp, s), "gemm")  # leaves X quantized in xq / xs
        fq = eng.lib.j4q_quant_matmul_q8_into

    def enqueue(i):
        if variant == "int8q":
            rc = fq(handles[i % copies], xqp, xsp, m, yp, s)
        else:
            rc = fn(handles[i % copies], xp, m, v, xqp, xsp, yp, s)
        if rc:
            check(rc, "gemm")

    # us_per_call from a region with events at its ends only; median / min / p90 from a second
    # region split into SAMPLES parts (each inner event adds a gap to the stream), as for the GEMVs
    _, _, _, host_us, _ = eng.time_region(enqueue, warmup)
    ms, _, _, _, host_bound = eng.time_region(enqueue, steps, host_us)
    _, sms, cnt, _, _ = eng.time_region(enqueue, steps, host_us, SAMPLES)
    per = ms / steps
    ops = 2.0 * m * n * k
    tops = ops / (per * 1e-3) / 1e12
    peak = BF16_PEAK_TFLOPS if variant == "bf16" else INT8_PEAK_TOPS
    for w in ws:
        eng.be.release(w)
    for p in (x, xq, xs, y):
        eng.hip.free(p)
    st = stats_us(sms, cnt)
    name = f"{qt.name.lower()}_gemm_{variant}_m{m}" + ("" if qt == QuantType.Q8_0 else f"_n{n}_k{k}")
    log(f"{name}: {per * 1e3:.2f} us (median {st['median_us']}), {tops:.0f} TOPS "
        f"({100 * tops / INT8_PEAK_TOPS:.1f}% of int8 peak, {100 * tops / peak:.1f}% of {variant} peak)")
    return {
        "workload": name,
        "quant": qt.name,
        "variant": variant,
        "M": m,
        "N": n,
        "K": k,
        "weight_copies": copies,
        "us_per_call": round(per * 1e3, 3),
        **st,
        "TOPS": round(tops, 1),
        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
        "frac_variant_peak": round(tops / peak, 4),
        "host_bound": host_bound,
    }


def gemm_regions(eng: Engine, m: int, variant: str, steps_list=(20, 40, 75, 200), idle_us: int = 50_000):
    """The Q8_0 GEMM of configs[3] at M = m in regions of back-to-back calls (steps_list), each
    after `idle_us` of a one-workgroup spin (the matrix cores idle), with events at the quarters
    of each region: how the time per call moves with the length of a sustained run."""
    n = k = 4096
    qt = QuantType.Q8_0
    copies = max(1, math.ceil(ROTATE_BYTES / qt.byte_size_for(n * k)))
    ws = [eng.weights(qt, n, k, 0x5EED8 + 31 * i)[0] for i in range(copies)]
    x = eng.bf16(m * k, 0x5EED9)
    xq, xs, y = eng.hip.malloc(m * k), eng.hip.malloc(4 * m * (k // 32)), eng.hip.malloc(4 * m * n)
    handles = [w.handle for w in ws]
    fn = eng.lib.j4q_quant_matmul_into
    v = N.GEMM_INT8 if variant == "int8" else N.GEMM_BF16
    s = C.c_void_p(eng.stream)
    xp, xqp, xsp, yp = C.c_void_p(x), C.c_void_p(xq), C.c_void_p(xs), C.c_void_p(y)

    def enqueue(i):
        rc = fn(handles[i % copies], xp, m, v, xqp, xsp, yp, s)
        if rc:
            check(rc, "gemm")

    _, _, _, host_us, _ = eng.time_region(enqueue, 10)
    out = []
    for calls in steps_list:
        check(eng.lib.j4q_spin(idle_us, s), "spin")
        ms, sms, cnt, _, _ = eng.time_region(enqueue, calls, host_us, 4)
        quarters = [round(1e3 * t / c, 2) for t, c in zip(sms, cnt)]
        out.append({"calls": calls, "us_per_call": round(1e3 * ms / calls, 2), "quarters_us": quarters})
        log(f"gemm {variant} M={m}, region of {calls} calls: {1e3 * ms / calls:.2f} us per call; quarters {quarters}")
    for w in ws:
        eng.be.release(w)
    for p in (x, xq, xs, y):
        eng.hip.free(p)
    return {"workload": f"q8_0_gemm_{variant}_m{m}", "idle_us_before_each": idle_us, "regions": out}


def timeline_workload(eng: Engine, name: str, qt: QuantType, rows: int, cols: int, parts=None, launches: int = 40):
    """Per-wave timeline of one batch-1 GEMV launch (j4q_gemv_trace): `launches` back-to-back
    launches over rotating weight copies, the last one traced. Reports, in us from the first
    wave's start, when waves start, when their x image is staged, when they finish, and how
    long x staging and each wave's items took (percentiles over the waves), by items per wave."""
    blob_bytes = qt.byte_size_for(rows * cols)
    copies = max(2, math.ceil(ROTATE_BYTES / blob_bytes))
    ws = []
    for i in range(copies):
        if parts:
            ps = [eng.weights(qt, r, cols, 0x71E + 97 * i + j)[0] for j, r in enumerate(parts)]
            ws.append(eng.be.concat_rows(ps))
            for p in ps:
                eng.be.release(p)
        else:
            ws.append(eng.weights(qt, rows, cols, 0x71E + 97 * i)[0])
    x = eng.f32(cols, 0x71F)
    y = eng.hip.malloc(4 * rows)
    max_waves = 16 * eng.info["compute_units"] * 8
    words = 4 * max_waves
    buf = eng.hip.malloc(8 * words)
    eng.hip.ok(eng.hip.h.hipMemset(C.c_void_p(buf), 0, 8 * words), "hipMemset")
    fn = eng.lib.j4q_quant_matvec_into
    s = C.c_void_p(eng.stream)

    def enqueue(i):
        check(fn(ws[i % copies].handle, C.c_void_p(x), None, C.c_void_p(y), 1, s), name)

    eng.time_region(enqueue, 5)
    # every launch of the region overwrites the trace: the last one's stamps remain
    check(eng.lib.j4q_gemv_trace(C.c_void_p(buf), words), "gemv_trace")
    ms, _, _, _, _ = eng.time_region(enqueue, launches)
    check(eng.lib.j4q_gemv_trace(None, 0), "gemv_trace")
    host = (C.c_uint64 * words)()
    eng.hip.ok(eng.hip.h.hipMemcpy(host, C.c_void_p(buf), 8 * words, 2), "hipMemcpy")
    for w in ws:
        eng.be.release(w)
    for p in (x, y, buf):
        eng.hip.free(p)
    rec = [(host[4 * i], host[4 * i + 1], host[4 * i + 2], host[4 * i + 3] & 0xFFFFFFFF) for i in range(max_waves)]
    rec = [r for r in rec if r[0]]
    return name, ms / launches, rec


def summarize_timeline(name, ms_per_launch, rec, ticks_per_us):
    t0 = min(r[0] for r in rec)
    start = sorted((r[0] - t0) / ticks_per_us for r in rec)
    staged = sorted((r[1] - t0) / ticks_per_us for r in rec)
    end = sorted((r[2] - t0) / ticks_per_us for r in rec)
    xdur = sorted((r[1] - r[0]) / ticks_per_us for r in rec)
    work = sorted((r[2] - r[1]) / ticks_per_us for r in rec)

    def pct(v):
        k = len(v)
        return {f"p{q}": round(v[min(k - 1, int(q * k / 100))], 2) for q in (0, 10, 50, 90, 100)}

    by_items = {}
    for it in sorted({r[3] for r in rec}):
        e = sorted((r[2] - t0) / ticks_per_us for r in rec if r[3] == it)
        by_items[str(it)] = {"waves": len(e), "end_us": pct(e)}
    out = {"workload": name, "us_per_launch": round(1e3 * ms_per_launch, 3), "waves": len(rec), "start_us": pct(start),
           "x_staged_us": pct(staged), "x_staging_us": pct(xdur), "work_us": pct(work), "end_us": pct(end),
           "end_by_items": by_items}
    log(f"timeline {name}: {out['us_per_launch']} us/launch, {len(rec)} waves; start {pct(start)}; "
        f"x staged {pct(staged)}; end {pct(end)}")
    return out


# Sizes of the streaming-read calibration: the algorithmic bytes of configs[0], [1], [2] (Q4_K,
# Q6_K), the fused gate|up matrix and the output head.
CALIBRATION_BYTES = [17858560, 25422848, 33103872, 48242688, 66060288, 430940160]


def torch_sum_reader(sizes, steps: int, warmup: int) -> None:
    """An independent reader (--torch-reader): torch.sum over rotating fp32 tensors of each size
    (at least ROTATE_BYTES of copies, as the GEMV workloads rotate), PyTorch's own reduction
    kernel, timed with events on torch's stream; prints one JSON list. It runs in a process of
    its own that never loads the engine: PyTorch's wheel ships its own HIP and HSA runtimes,
    and a process holding both those and the engine's (ROCm's) crashed under rocprofv3 at
    torch's first kernel launch. A Python loop launches the sums, so the events include any
    host gap between launches; the rocprofv3 kernel trace gives the kernel durations alone."""
    import torch

    out = []
    for nb in sizes:
        copies = max(1, math.ceil(ROTATE_BYTES / nb))
        bufs = [torch.ones(nb // 4, device="cuda") for _ in range(copies)]
        outs = torch.empty(copies, device="cuda")
        for i in range(warmup):
            torch.sum(bufs[i % copies], dim=0, out=outs[i % copies])
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            torch.sum(bufs[i % copies], dim=0, out=outs[i % copies])
        b.record()
        torch.cuda.synchronize()
        us = 1e3 * a.elapsed_time(b) / steps
        del bufs
        out.append({"bytes": nb, "copies": copies, "us_per_launch": round(us, 3),
                    "GBps": round(nb / (us * 1e-6) / 1e9, 1),
                    "note": "event-timed Python loop: an upper bound on the kernel time"})
    print(json.dumps(out), flush=True)


def run_torch_reader(sizes, steps: int, warmup: int):
    """torch_sum_reader in a child process (see there); its JSON list, or None if it failed."""
    import subprocess

    cmd = [sys.executable, os.path.abspath(__file__), "--torch-reader", ",".join(map(str, sizes)),
           "--steps", str(steps), "--warmup", str(warmup)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=600)
    if proc.returncode != 0:
        err = [l for l in proc.stderr.splitlines() if l.strip() and not l.startswith(("W20", "E20", "I20"))]
        log(f"warning: torch reader exited with {proc.returncode}: " + " | ".join(err[-6:]))
        return None
    return json.loads(proc.stdout.strip().splitlines()[-1])


def calibrate(eng: Engine, steps: int, warmup: int):
    """The practical HBM read ceiling of one launch of each size (j4q_stream_read over rotating
    buffers, so the Infinity Cache cannot serve them: 1 or 2 workgroups per CU, 4 or 8 1 KB
    loads in flight per wave), PyTorch's torch.sum over the same sizes as an independent
    reader, and a copy kernel of known size so a counter profile of this process can scale
    the GEMV's byte counters."""
    out = []
    for nbytes in CALIBRATION_BYTES:
        nb = (nbytes + 15) // 16 * 16
        copies = max(1, math.ceil(ROTATE_BYTES / nb))
        bufs = [eng.hip.malloc(nb) for _ in range(copies)]
        sink = eng.hip.malloc(4 * 4 * eng.info["compute_units"])
        row = {"workload": f"stream_read_{nb}", "bytes": nb, "copies": copies}
        for wpc, depth in ((1, 4), (2, 4), (1, 8), (2, 8)):
            fn = eng.lib.j4q_stream_read
            s = C.c_void_p(eng.stream)

            def enqueue(i):
                rc = fn(C.c_void_p(bufs[i % copies]), nb, C.c_void_p(sink), wpc, depth, s)
                if rc:
                    check(rc, "stream_read")

            eng.time_region(enqueue, warmup)
            ms, _, _, _, _ = eng.time_region(enqueue, steps)
            _, sms, cnt, _, _ = eng.time_region(enqueue, steps, 30.0, SAMPLES)
            st = stats_us(sms, cnt)
            row[f"wg_per_cu_{wpc}_depth_{depth}"] = {"us_per_launch": round(1e3 * ms / steps, 3), "sampled": st,
                                                     "GBps": round(nb / (ms / steps * 1e-3) / 1e9, 1)}
        for b in bufs + [sink]:
            eng.hip.free(b)
        best = max(v["GBps"] for k, v in row.items() if k.startswith("wg_per_cu"))
        row["best_GBps"] = best
        log(f"stream_read {nb / 1e6:.1f} MB: {best:.0f} GB/s ({100 * best / HBM_PEAK_GBS:.1f}% of HBM peak)")
        out.append(row)
    sums = run_torch_reader([r["bytes"] for r in out], steps, warmup)
    for row, t in zip(out, sums or []):
        row["torch_sum"] = t
        log(f"torch.sum {row['bytes'] / 1e6:.1f} MB: {t['GBps']:.0f} GB/s (event-timed, separate process)")
    n = 256 << 20
    src, dst = eng.hip.malloc(n), eng.hip.malloc(n)
    for _ in range(3):
        check(eng.lib.j4q_copy(C.c_void_p(dst), C.c_void_p(src), n, C.c_void_p(eng.stream)), "copy")
    eng.hip.sync()
    eng.hip.free(src)
    eng.hip.free(dst)
    log(f"calibration copy: 3 x {n} bytes")
    return out


def measured_traffic(workload: str):
    """HBM bytes per launch of a workload's kernel from the committed counter profile
    (profiles/gemv_traffic.json: FETCH_SIZE and WRITE_SIZE passes scaled by a copy kernel of
    known size), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t.get("workloads", {}).get(workload, {}).get("traffic_bytes_per_launch")


def host_description():
    model, mhz = "unknown", None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            if line.startswith("cpu MHz") and mhz is None:
                mhz = float(line.split(":", 1)[1])
    except OSError:
        pass
    try:
        with open("/sys/devices/system/cpu/cpu0/cpufreq/scaling_max_freq") as f:
            max_mhz = int(f.read()) / 1e3
    except (OSError, ValueError):
        max_mhz = None
    return {"cpu_model": model, "cpu_mhz_now": mhz, "cpu_mhz_max": max_mhz, "nproc": os.cpu_count()}


def cpu_rows(seconds: float):
    """The reference's CPU algorithm and the oracle's restated loops, each on one pinned host
    core over a bounded sample of a config (the oracle is the checker elsewhere; here it is
    the timed CPU baseline). Returns (headline row for configs[4] B = 1, all rows)."""
    import numpy as np

    import oracle
    from jax4j_amd import synthetic as S

    def timed(fn, budget):
        fn()  # warm
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return el / reps, reps

    old = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {min(old)})
    rows = []
    try:
        budget = max(0.5, seconds / 8)
        gemvs = [
            ("configs[0] Q8_0 GEMV 4096x4096", QuantType.Q8_0, 4096, 4096, "restated ggml dequantize_row_q8_0 + float dot (no reference CPU path: CpuBackend.java:698-701 rejects Q8_0)"),
            ("configs[1] Q4_0 GEMV 11008x4096 B=1", QuantType.Q4_0, 11008, 4096, "restated CpuQ4Gemm.multiply (CpuQ4Gemm.java:26-46), the reference's algorithm"),
            ("configs[2] Q4_K GEMV 14336x4096", Q4K, 14336, 4096, "restated ggml dequantize_row_q4_K + float dot (no reference CPU path)"),
            ("configs[2] Q6_K GEMV 4096x14336", Q6K, 4096, 14336, "restated ggml dequantize_row_q6_K + float dot (no reference CPU path)"),
        ]
        per_gemv = {}
        for name, qt, n, k, how in gemvs:
            blob = S.quant_blocks(qt, 0x5EED5, n, k)
            x = S.activations_f32(0x5EED6, k)
            fn = (lambda b=blob, n=n, k=k, x=x: oracle.q4_0_multiply(b, n, k, x)) if qt == QuantType.Q4_0 else \
                 (lambda b=blob, qt=qt, n=n, k=k, x=x: oracle.matvec(qt.id, b, n, k, x))
            t, reps = timed(fn, budget)
            per_gemv[(qt, n, k)] = t
            alg = blob.nbytes + 4 * k + 4 * n
            rows.append({"config": name, "cores": 1, "kind": "port", "algorithm": how, "ms_per_call": round(t * 1e3, 2),
                         "GBps": round(alg / t / 1e9, 3), "sample": f"full matrix, batch 1, {reps} reps"})
        rows.append({"config": "configs[1] Q4_0 GEMV 11008x4096 B=8", "cores": 1, "kind": "port",
                     "algorithm": "8 calls of the restated CpuQ4Gemm.multiply (the SPI is matrix x vector)",
                     "ms_per_call": round(8e3 * per_gemv[(QuantType.Q4_0, 11008, 4096)], 2),
                     "GBps": round((25362432 + 8 * 4 * (4096 + 11008)) / (8 * per_gemv[(QuantType.Q4_0, 11008, 4096)]) / 1e9, 3),
                     "sample": "derived from the B=1 timing x 8"})
        # the oracle's exact product (fp64 accumulation over the dequantized W and
        # bf16 X) on a 32-row slice of X; ops/s scale with M, so the rate holds for every M
        m, n, k = 32, 4096, 4096
        wblob = S.quant_blocks(QuantType.Q8_0, 0x5EED8, n, k)
        xb = S.activations_bf16(0x5EED9, m * k)
        t, reps = timed(lambda: oracle.gemm_f64(xb, wblob, m, n, k), budget)
        rows.append({"config": "configs[3] Q8_0 GEMM N=K=4096", "cores": 1, "kind": "port",
                     "algorithm": "restated scalar product of bf16 X and the dequantized W (fp64 accumulation); the reference has no GEMM",
                     "ms_per_call": round(t * 1e3, 2), "TOPS": round(2 * m * n * k / t / 1e12, 5),
                     "sample": f"M = 32 rows of X, {reps} reps"})
        # one decoder layer's seven GEMVs and the head, extrapolated to 32 layers
        layer_s = 0.0
        for name, qt, n, k in LLAMA3_8B_LAYER:
            layer_s += per_gemv.get((qt, n, k)) or timed(
                lambda qt=qt, n=n, k=k, b=S.quant_blocks(qt, 7, n, k), x=S.activations_f32(8, k): oracle.matvec(qt.id, b, n, k, x),
                0.2)[0]
        hq, hn, hk = LLAMA3_8B_HEAD
        hblob = S.quant_blocks(hq, 9, hn, hk)
        hx = S.activations_f32(10, hk)
        head_s, _ = timed(lambda: oracle.matvec(hq.id, hblob, hn, hk, hx), 0.1)
        step_s = 32 * layer_s + head_s
        weights = 32 * sum(qt.byte_size_for(n * k) for _, qt, n, k in LLAMA3_8B_LAYER) + hq.byte_size_for(hn * hk)
        head_row = {
            "value": round(weights / step_s / 1e9, 3),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": (f"oracle/quant_ref.c restated ggml Q4_K/Q6_K loops (no reference CPU path for these types; the "
                       f"reference's own CpuQ4Gemm runs Q4_0 at the rate in cpu_rows): one decoder layer's 7 GEMVs "
                       f"({layer_s * 1e3:.0f} ms) and the 128256x4096 Q6_K head ({head_s * 1e3:.0f} ms) timed on one "
                       f"pinned core, step = 32 x layer + head = {step_s:.2f} s ({1 / step_s:.3f} tok/s)"),
        }
        rows.append({"config": "configs[4] decode step B=1", "cores": 1, "kind": "port",
                     "algorithm": "sum of the restated GEMVs", "ms_per_step": round(step_s * 1e3, 1),
                     "GBps": head_row["value"], "tokens_per_s": round(1 / step_s, 4),
                     "sample": "one layer + head timed, extrapolated to 32 layers"})
        rows.append({"config": "jax4j-simd", "cores": 0, "kind": "n/a",
                     "algorithm": "not applicable: jax4j-simd is an AAD replay engine with no quantized matmul"})
    finally:
        os.sched_setaffinity(0, old)
    return head_row, rows


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=75)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline workload only, no CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="", help="comma list of workload groups to run: gemv,gemm,decode (default all)")
    ap.add_argument("--batches", default="4,8,16", help="comma list of batch sizes for the batched decode-step lines")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run the streaming-read ceiling and a copy kernel of known size (counter scaling)")
    ap.add_argument("--torch-reader", default="", metavar="BYTES,...",
                    help="only run PyTorch's torch.sum over rotating tensors of these sizes, in this process "
                         "(--calibrate runs it as a child process)")
    ap.add_argument("--gemm-regions", action="store_true",
                    help="also time the bf16 and int8 Q8_0 GEMM at M = 2048 and 512 in regions of 20 to 200 calls "
                         "after an idle spin (time per call against the length of a sustained run)")
    ap.add_argument("--resident", action="store_true",
                    help="also time the decode step's four B = 1 GEMV shapes with one weight copy launched back to "
                         "back (the weights stay in the 256 MB Infinity Cache) beside the same shapes over "
                         "rotating copies: how much of each launch HBM accounts for")
    ap.add_argument("--timeline", action="store_true",
                    help="also record the per-wave timeline of one launch of the dominant GEMV and of the step's "
                         "smaller B = 1 GEMVs (j4q_gemv_trace)")
    args = ap.parse_args()
    if args.torch_reader:
        torch_sum_reader([int(b) for b in args.torch_reader.split(",") if b], args.steps, args.warmup)
        return
    if args.gpus != 1:
        print(
            f"bench.py: this engine is measured on one GPU; --gpus {args.gpus} is not supported "
            "(across GPUs the path would shard the GEMV rows, gather y and replicate x)",
            file=sys.stderr,
        )
        sys.exit(2)

    eng = Engine()
    log(f"device {eng.info['name']} {eng.info['arch']} CUs={eng.info['compute_units']} "
        f"sclk={eng.info['max_clock_khz'] / 1e3:.0f} MHz HBM={eng.info['hbm_bytes'] / 2**30:.0f} GiB")

    groups = set(filter(None, args.only.split(","))) or {"gemv", "gemm", "decode"}
    model = DecodeModel(eng)
    log(f"configs[4] weights: {model.total} bytes in HBM")
    head = decode_workload(eng, model, 1, args.steps, args.warmup)
    others = []
    if not args.quick:
        if "decode" in groups:
            for batch in [int(b) for b in args.batches.split(",") if b]:
                others.append(decode_workload(eng, model, batch, max(2, args.steps // 2), max(1, args.warmup // 2)))
            others.append(decode_workload(eng, model, 1, max(2, args.steps // 4), 2, plan=False))
    model.release()
    dominant = gemv_workload(eng, DOMINANT, Q4K, 28672, 4096, 1, args.steps, args.warmup, parts=[14336, 14336])
    cal = calibrate(eng, args.steps, args.warmup) if args.calibrate else None
    regions = None
    if args.gemm_regions:
        regions = [gemm_regions(eng, m, var) for m, var in ((2048, "bf16"), (2048, "int8"), (512, "bf16"))]
    resident = None
    if args.resident:
        resident = []
        for name, qt, n, k, parts in STEP_SHAPES_B1:
            rot = gemv_workload(eng, name, qt, n, k, 1, args.steps, args.warmup, parts)
            res = gemv_workload(eng, name + "_resident", qt, n, k, 1, args.steps, args.warmup, parts, rotate_bytes=1)
            resident.append({"workload": name, "us_per_launch_rotating": rot["us_per_launch"],
                             "us_per_launch_resident": res["us_per_launch"],
                             "median_us_rotating": rot["sampled"]["median_us"],
                             "median_us_resident": res["sampled"]["median_us"]})
    timeline = None
    if args.timeline:
        khz = C.c_int()
        eng.hip.ok(eng.hip.h.hipDeviceGetAttribute(C.byref(khz), HIP_ATTR_WALL_CLOCK_RATE, 0), "hipDeviceGetAttribute")
        tpu = khz.value / 1e3
        timeline = [summarize_timeline(*timeline_workload(eng, *w), tpu) for w in STEP_SHAPES_B1]
    if not args.quick:
        if "gemv" in groups:
            others.append(gemv_workload(eng, "q4_0_gemv_b1", QuantType.Q4_0, 11008, 4096, 1, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q4_0_gemv_b8", QuantType.Q4_0, 11008, 4096, 8, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q8_0_gemv_b1", QuantType.Q8_0, 4096, 4096, 1, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q4_k_gemv_gate_up", Q4K, 14336, 4096, 1, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q6_k_gemv_down", Q6K, 4096, 14336, 1, args.steps, args.warmup))
        if "gemm" in groups:
            for m in (32, 128, 512, 2048):
                for variant in ("int8", "bf16"):
                    others.append(gemm_workload(eng, m, variant, args.steps, args.warmup))
            # the int8 GEMM on X quantized once (one X feeding several Q8_0 matrices)
            for m in (512, 2048):
                others.append(gemm_workload(eng, m, "int8q", args.steps, args.warmup))
            # the prefill GEMM over the K-quant matrices of configs[2] and the Q4_0 one of configs[1]
            for qt, n, k in ((Q4K, 14336, 4096), (Q6K, 4096, 14336), (QuantType.Q4_0, 11008, 4096)):
                for m in ((32, 512, 2048) if qt != QuantType.Q4_0 else (512,)):
                    others.append(gemm_workload(eng, m, "bf16", max(2, args.steps // 2), max(1, args.warmup // 2),
                                                n=n, k=k, qt=qt))

    cpu, cpu_all = (None, None) if (args.quick or args.only) else cpu_rows(args.cpu_seconds)
    achieved = dominant["GBps"]
    out = {
        "metric": METRIC,
        "value": head["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded GGUF blocks with the benchmark distributions, random-init weights of the named "
                "shapes, generated in HBM)",
        "config": {
            "workload": "configs[4]: Llama-3-8B-shaped decode step, matmuls only, Q4_K_M mix (32 x q/k/v/o/gate/up "
                        "Q4_K + down Q6_K, 128256x4096 Q6_K head), batch 1, through the decode plan (q|k|v and "
                        "gate|up fused, residual quantMatvecAdd in place, one HIP graph per step)",
            "layers": 32,
            "batch": 1,
            "weight_bytes_per_step": model.total,
            "gemvs_per_step": head["gemvs_per_step"],
            "tokens_per_s": head["tokens_per_s"],
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{DOMINANT}: the step's dominant kernel, gemv_kernel<Q4_K> over the fused 28672x4096 gate|up "
                      f"matrix, {dominant['algorithmic_bytes']} algorithmic bytes per launch",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(DOMINANT),
        },
        "cpu_baseline": cpu,
        "stats": {k: head[k] for k in ("median_ms", "min_ms", "p90_ms", "samples")},
        "workloads": [head, dominant] + others,
        "cpu_rows": cpu_all,
        "calibration": cal,
        "timeline": timeline,
        "gemm_regions": regions,
        "resident": resident,
        "host": host_description(),
        "device": eng.info,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

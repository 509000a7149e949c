#!/usr/bin/env python3
"""Benchmark of the MI355X GGUF quantized-matmul engine (one GPU).

A "step" is one pass of the hot path over one batch of synthetic input: one GEMV launch
for the GEMV workloads, one prefill GEMM for the GEMM ones, and the 225 GEMVs of a
Llama-3-8B-shaped decode step for the decode workloads. The headline workload (`value`)
is the benchmark's configs[1]: Q4_0 GEMV, N=11008, K=4096, batch 1, in HBM GB/s of
algorithmic bytes (weight blob + x + y per launch).

Measurement: inputs are resident in HBM before timing. Each GEMV workload rotates over
>= 512 MB of distinct weight copies so the 256 MB Infinity Cache cannot serve them. A
bounded spin kernel holds the engine stream while the host queues the timed launches, so
they execute back to back; HIP events on that same stream bracket exactly the K timed
launches (warmup launches run first, untimed).

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
# HBM bytes per launch of the headline kernel, measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
# counters scaled by a copy kernel of known size (written from those runs; see the .md beside it).
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_q4_0_n11008_k4096_b1_traffic.json")


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
            "hipStreamBeginCapture": [C.c_void_p, C.c_int],
            "hipStreamEndCapture": [C.c_void_p, C.POINTER(C.c_void_p)],
            "hipGraphInstantiate": [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t],
            "hipGraphLaunch": [C.c_void_p, C.c_void_p],
            "hipGraphExecDestroy": [C.c_void_p],
            "hipGraphDestroy": [C.c_void_p],
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

    def record(self, e: int, stream: int) -> None:
        self.ok(self.h.hipEventRecord(C.c_void_p(e), C.c_void_p(stream)), "hipEventRecord")

    def capture(self, stream: int, enqueue):
        """A graph of everything `enqueue()` puts on `stream` (relaxed capture mode)."""
        self.ok(self.h.hipStreamBeginCapture(C.c_void_p(stream), 2), "hipStreamBeginCapture")
        try:
            enqueue()
        finally:
            g = C.c_void_p()
            self.ok(self.h.hipStreamEndCapture(C.c_void_p(stream), C.byref(g)), "hipStreamEndCapture")
        ex = C.c_void_p()
        self.ok(self.h.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return ex.value, g.value

    def graph_launch(self, exec_: int, stream: int) -> None:
        self.ok(self.h.hipGraphLaunch(C.c_void_p(exec_), C.c_void_p(stream)), "hipGraphLaunch")

    def graph_free(self, exec_: int, graph: int) -> None:
        self.ok(self.h.hipGraphExecDestroy(C.c_void_p(exec_)), "hipGraphExecDestroy")
        self.ok(self.h.hipGraphDestroy(C.c_void_p(graph)), "hipGraphDestroy")

    def elapsed_ms(self, a: int, b: int) -> float:
        self.ok(self.h.hipEventSynchronize(C.c_void_p(b)), "hipEventSynchronize")
        ms = C.c_float()
        self.ok(self.h.hipEventElapsedTime(C.byref(ms), C.c_void_p(a), C.c_void_p(b)), "hipEventElapsedTime")
        return float(ms.value)


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

    def time_region(self, enqueue, launches: int, host_us_per_launch: float = 30.0):
        """GPU time (ms) of `launches` launches queued by `enqueue(i)` behind a spin kernel
        long enough for the host to queue them all, and the host's own queueing time (us
        per launch). If the host was slower than the spin, the GPU may have idled and the
        region is flagged host-bound."""
        self.hip.sync()
        e0, e1 = self.hip.event(), self.hip.event()
        spin_us = int(min(5_000_000, 3000 + 1.5 * launches * host_us_per_launch))
        check(self.lib.j4q_spin(spin_us, C.c_void_p(self.stream)), "spin")
        self.hip.record(e0, self.stream)
        t0 = time.perf_counter()
        for i in range(launches):
            enqueue(i)
        host_us = (time.perf_counter() - t0) * 1e6
        self.hip.record(e1, self.stream)
        ms = self.hip.elapsed_ms(e0, e1)
        self.hip.sync()
        if host_us > spin_us:
            log(f"warning: host queueing ({host_us:.0f} us) outlasted the spin ({spin_us} us); region may be host-bound")
        return ms, host_us / max(launches, 1), host_us > spin_us


def gemv_workload(eng: Engine, name: str, qt: QuantType, rows: int, cols: int, batch: int, steps: int, warmup: int):
    blob_bytes = qt.byte_size_for(rows * cols)
    copies = max(1, math.ceil(ROTATE_BYTES / blob_bytes))
    log(f"{name}: {qt.name} N={rows} K={cols} B={batch}, {copies} weight copies")
    ws = [eng.weights(qt, rows, cols, 0x5EED5 + 97 * i)[0] for i in range(copies)]
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

    _, host_us, _ = eng.time_region(enqueue, warmup)
    ms, _, host_bound = eng.time_region(enqueue, steps, host_us)
    per = ms / steps
    alg = blob_bytes + 4 * batch * cols + 4 * batch * rows
    gbs = alg / (per * 1e-3) / 1e9
    for w in ws:
        eng.be.release(w)
    eng.hip.free(x)
    eng.hip.free(y)
    log(f"{name}: {per * 1e3:.2f} us/launch, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
    return {
        "workload": name,
        "quant": qt.name,
        "N": rows,
        "K": cols,
        "batch": batch,
        "weight_copies": copies,
        "us_per_launch": round(per * 1e3, 3),
        "algorithmic_bytes": alg,
        "GBps": round(gbs, 1),
        "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "host_bound": host_bound,
    }


def decode_workload(eng: Engine, batch: int, steps: int, warmup: int, layers: int = 32, fused: bool = False,
                    graph: bool = False):
    """Synthetic Llama-3-8B decode step, matmuls only (Q4_K_M mix): 32 x (q, k, v, o, gate,
    up: Q4_K; down: Q6_K) + a 128256 x 4096 Q6_K head = 225 GEMVs per step. With `fused`,
    the matrices that share an input run as one (q|k|v 6144 x 4096, gate|up 28672 x 4096, the
    rows concatenated as j4q_concat_rows does at load time): 129 launches streaming the same
    bytes. With `graph`, one step is captured in a HIP graph and replayed."""
    if fused:
        shapes = [(QuantType.Q4_K, 6144, 4096), (QuantType.Q4_K, 4096, 4096), (QuantType.Q4_K, 28672, 4096),
                  (QuantType.Q6_K, 4096, 14336)]
    else:
        shapes = [(QuantType.Q4_K, 4096, 4096), (QuantType.Q4_K, 1024, 4096), (QuantType.Q4_K, 1024, 4096),
                  (QuantType.Q4_K, 4096, 4096), (QuantType.Q4_K, 14336, 4096), (QuantType.Q4_K, 14336, 4096),
                  (QuantType.Q6_K, 4096, 14336)]
    mats, total = [], 0
    seed = 0xDEC0DE
    for layer in range(layers):
        for qt, n, k in shapes:
            w, nb = eng.weights(qt, n, k, seed)
            seed += 1
            mats.append((w, n, k))
            total += nb
    w, nb = eng.weights(QuantType.Q6_K, 128256, 4096, seed)
    mats.append((w, 128256, 4096))
    total += nb
    x4 = eng.f32(batch * 4096, 0xA11)
    x14 = eng.f32(batch * 14336, 0xA12)
    y = eng.hip.malloc(4 * batch * 128256)
    fn = eng.lib.j4q_quant_matvec_into
    s = C.c_void_p(eng.stream)
    launches = [(w.handle, C.c_void_p(x14 if k == 14336 else x4)) for (w, n, k) in mats]
    yp = C.c_void_p(y)

    def one_step():
        for h, xp in launches:
            rc = fn(h, xp, None, yp, batch, s)
            if rc:
                check(rc, "decode")

    g = None
    if graph:
        g = eng.hip.capture(eng.stream, one_step)

        def enqueue(step):
            eng.hip.graph_launch(g[0], eng.stream)
    else:
        def enqueue(step):
            one_step()

    _, host_us, _ = eng.time_region(enqueue, warmup, 30.0 * len(launches))
    ms, _, host_bound = eng.time_region(enqueue, steps, host_us)
    per = ms / steps
    if g:
        eng.hip.graph_free(*g)
    for (w, _, _) in mats:
        eng.be.release(w)
    for p in (x4, x14, y):
        eng.hip.free(p)
    gbs = total / (per * 1e-3) / 1e9
    tag = ("fused" if fused else "unfused") + ("+graph" if graph else "")
    log(f"decode B={batch} {tag}: {per:.3f} ms/step, {gbs:.0f} GB/s weights, {batch / (per * 1e-3):.0f} tok/s")
    return {
        "workload": f"llama3-8b decode step B={batch} {tag}",
        "gemvs_per_step": len(launches),
        "batch": batch,
        "ms_per_step": round(per, 4),
        "weight_bytes_per_step": total,
        "GBps": round(gbs, 1),
        "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(batch / (per * 1e-3), 1),
        "host_bound": host_bound,
    }


def gemm_workload(eng: Engine, m: int, variant: str, steps: int, warmup: int, n: int = 4096, k: int = 4096):
    """Q8_0 prefill GEMM Y[m, n] = X[m, k] . W^T with bf16 X; the int8 variant's
    timed call includes quantizing X (j4q_quant_matmul_into runs both kernels)."""
    qt = QuantType.Q8_0
    blob_bytes = qt.byte_size_for(n * k)
    copies = max(1, math.ceil(ROTATE_BYTES / blob_bytes))
    ws = [eng.weights(qt, n, k, 0x5EED8 + 31 * i)[0] for i in range(copies)]
    x = eng.bf16(m * k, 0x5EED9)
    xq = eng.hip.malloc(m * k)
    xs = eng.hip.malloc(4 * m * (k // 32))
    y = eng.hip.malloc(4 * m * n)
    handles = [w.handle for w in ws]
    fn = eng.lib.j4q_quant_matmul_into
    v = N.GEMM_INT8 if variant == "int8" else N.GEMM_BF16
    s = C.c_void_p(eng.stream)
    xp, xqp, xsp, yp = C.c_void_p(x), C.c_void_p(xq), C.c_void_p(xs), C.c_void_p(y)

    def enqueue(i):
        rc = fn(handles[i % copies], xp, m, v, xqp, xsp, yp, s)
        if rc:
            check(rc, "gemm")

    _, host_us, _ = eng.time_region(enqueue, warmup)
    ms, _, host_bound = eng.time_region(enqueue, steps, host_us)
    per = ms / steps
    ops = 2.0 * m * n * k
    tops = ops / (per * 1e-3) / 1e12
    peak = INT8_PEAK_TOPS if variant == "int8" else BF16_PEAK_TFLOPS
    for w in ws:
        eng.be.release(w)
    for p in (x, xq, xs, y):
        eng.hip.free(p)
    log(f"gemm {variant} M={m}: {per * 1e3:.2f} us, {tops:.0f} TOPS ({100 * tops / INT8_PEAK_TOPS:.1f}% of int8 peak, "
        f"{100 * tops / peak:.1f}% of {variant} peak)")
    return {
        "workload": f"q8_0_gemm_{variant}_m{m}",
        "variant": variant,
        "M": m,
        "N": n,
        "K": k,
        "weight_copies": copies,
        "us_per_call": round(per * 1e3, 3),
        "TOPS": round(tops, 1),
        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
        "frac_variant_peak": round(tops / peak, 4),
        "host_bound": host_bound,
    }


def calibrate_copy(eng: Engine, nbytes: int = 256 << 20, reps: int = 3) -> None:
    """Runs the engine's streaming copy kernel on `nbytes` a few times, so a counter profile of
    this process has a kernel of known traffic to scale the GEMV's byte counters by."""
    src, dst = eng.hip.malloc(nbytes), eng.hip.malloc(nbytes)
    for _ in range(reps):
        check(eng.lib.j4q_copy(C.c_void_p(dst), C.c_void_p(src), nbytes, C.c_void_p(eng.stream)), "copy")
    eng.hip.sync()
    eng.hip.free(src)
    eng.hip.free(dst)
    log(f"calibration copy: {reps} x {nbytes} bytes")


def measured_traffic(workload: str):
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t.get("traffic_bytes_per_launch") if t.get("workload") == workload else None


def cpu_baseline(seconds: float = 10.0):
    """The reference's CPU algorithm (CpuQ4Gemm.multiply, restated in C by the oracle) on the
    headline workload, single-threaded on one pinned host core."""
    import numpy as np

    import oracle
    from jax4j_amd import synthetic as S

    rows, cols = 11008, 4096
    blob = S.quant_blocks(QuantType.Q4_0, 0x5EED5, rows, cols)
    x = S.activations_f32(0x5EED6, cols)
    old = os.sched_getaffinity(0)
    core = min(old)
    os.sched_setaffinity(0, {core})
    try:
        oracle.q4_0_multiply(blob, rows, cols, x)  # warm
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.q4_0_multiply(blob, rows, cols, x)
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    finally:
        os.sched_setaffinity(0, old)
    per = el / reps
    alg = blob.nbytes + 4 * cols + 4 * rows
    cpu_model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(alg / per / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (
            f"oracle/quant_ref.c ref_q4_0_multiply (restated CpuQ4Gemm.multiply, -O2 -ffp-contract=off), "
            f"full Q4_0 {rows}x{cols} matrix, batch 1, {reps} reps in {el:.1f} s on one pinned core "
            f"({cpu_model}; host nproc={os.cpu_count()}); {per * 1e3:.1f} ms per GEMV"
        ),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline workload only, no CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="", help="comma list of workload groups to run: gemv,gemm,decode (default all)")
    ap.add_argument("--calibrate", action="store_true", help="also run a copy kernel of known size (for counter scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: this engine is measured on one GPU; --gpus {args.gpus} is not supported "
            "(the path would shard GEMV rows across GPUs, see DESIGN.md)",
            file=sys.stderr,
        )
        sys.exit(2)

    eng = Engine()
    log(f"device {eng.info['name']} {eng.info['arch']} CUs={eng.info['compute_units']} "
        f"sclk={eng.info['max_clock_khz'] / 1e3:.0f} MHz HBM={eng.info['hbm_bytes'] / 2**30:.0f} GiB")

    head = gemv_workload(eng, "q4_0_gemv_b1", QuantType.Q4_0, 11008, 4096, 1, args.steps, args.warmup)
    if args.calibrate:
        calibrate_copy(eng)
    others = []
    groups = set(filter(None, args.only.split(","))) or {"gemv", "gemm", "decode"}
    if not args.quick:
        if "gemv" in groups:
            others.append(gemv_workload(eng, "q4_0_gemv_b8", QuantType.Q4_0, 11008, 4096, 8, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q8_0_gemv_b1", QuantType.Q8_0, 4096, 4096, 1, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q4_k_gemv_gate_up", QuantType.Q4_K, 14336, 4096, 1, args.steps, args.warmup))
            others.append(gemv_workload(eng, "q6_k_gemv_down", QuantType.Q6_K, 4096, 14336, 1, args.steps, args.warmup))
        if "gemm" in groups:
            for m in (32, 128, 512, 2048):
                for variant in ("int8", "bf16"):
                    others.append(gemm_workload(eng, m, variant, max(10, args.steps // 2), max(5, args.warmup // 2)))
        if "decode" in groups:
            dsteps = max(2, min(20, args.steps // 10))
            others.append(decode_workload(eng, 1, dsteps, 2))
            others.append(decode_workload(eng, 1, dsteps, 2, fused=True))
            others.append(decode_workload(eng, 1, dsteps, 2, fused=True, graph=True))
            others.append(decode_workload(eng, 16, max(2, dsteps // 4), 1))
            others.append(decode_workload(eng, 16, max(2, dsteps // 4), 1, fused=True, graph=True))

    cpu = None if (args.quick or args.only) else cpu_baseline(args.cpu_seconds)
    per_ms = head["us_per_launch"] / 1e3
    achieved = head["GBps"]
    out = {
        "metric": METRIC,
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded GGUF blocks with the benchmark distributions, generated in HBM)",
        "config": {
            "workload": "configs[1]: Q4_0 GEMV N=11008 K=4096 batch 1 (fp32 x, fp32 accumulation)",
            "quant": "Q4_0",
            "N": 11008,
            "K": 4096,
            "batch": 1,
            "weight_copies_rotated": head["weight_copies"],
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("q4_0_gemv_b1"),
        },
        "cpu_baseline": cpu,
        "workloads": [head] + others,
        "device": eng.info,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

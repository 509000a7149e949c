"""Build recipe for the engine's C-ABI shared library (gfx950 only).

Compiles every ``csrc/*.hip`` with ``hipcc --offload-arch=gfx950`` into objects under
``jax4j_amd/_build/`` and links ``jax4j_amd/lib/libjax4j_mi355x.so``. Packed-FP32 VALU
instructions are disabled for all device code (``-packed-fp32-ops``).
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libjax4j_mi355x.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results and accumulator inputs in VGPRs: with accumulators in AGPRs the register
    # allocator rotated them through copies that each waited for the MFMA before, which
    # serialized the matrix pipe (19 instead of 44 cycles per 16x16x32 MFMA, measured)
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # the one atomic (a single lane's LDS add handing out row groups in the batch-1 GEMV) as a
    # plain ds_add_rtn: the atomic optimizer's lane-count rewrite waited for its result and
    # broadcast it right away, where the kernel reads it a group's worth of items later
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is expected.
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build_engine(jobs: int | None = None) -> Path:
    """Compile all HIP sources and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD / (s.stem + ".o") for s in sources]
    jobs = jobs or min(8, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    """Build the CPU oracle (test infrastructure) with its Makefile."""
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    return ROOT / "oracle" / "libquantref.so"


if __name__ == "__main__":
    print(build_engine())
    print(build_oracle())

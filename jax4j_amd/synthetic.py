"""Seeded synthetic inputs with the benchmark distributions (host side).

Thin wrappers over the engine library's host generator (``j4q_synth_*_host``), which shares
its code with the device generator, so a matrix generated here is byte-identical to one
generated in HBM with the same seed. Runs on any machine; no GPU needed.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _native as N
from .backend import check
from .tensor import QuantType


def quant_blocks(qtype: QuantType, seed: int, rows: int, cols: int) -> np.ndarray:
    """GGUF blocks (uint8) of a [rows, cols] matrix of ``qtype``."""
    nbytes = qtype.byte_size_for(rows * cols)
    out = np.empty(nbytes, dtype=np.uint8)
    check(N.load().j4q_synth_quant_host(qtype.id, seed, rows, cols, out.ctypes.data_as(C.c_void_p), nbytes), "synth")
    return out


def activations_f32(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(N.load().j4q_synth_f32_host(seed, n, out.ctypes.data_as(C.c_void_p)), "synth")
    return out


def activations_bf16(seed: int, n: int) -> np.ndarray:
    """bf16 bit patterns (uint16) of N(0,1) values."""
    out = np.empty(n, dtype=np.uint16)
    check(N.load().j4q_synth_bf16_host(seed, n, out.ctypes.data_as(C.c_void_p)), "synth")
    return out

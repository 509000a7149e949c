"""Writes kat_blocks.json: hand-derived known-answer blocks for every format.

Each case builds GGUF bytes from chosen element values following the published block
layouts (the reference's Q4_0/Q2_0 comments at CpuQ4Gemm.java:4-6 and CpuQ2Gemm.java:39-42;
ggml block_q8_0 / block_q4_K / block_q6_K for the rest) and records the values the
format defines in closed form: power-of-two scales make every expected value an exact
small multiple, so no decoder is involved in producing the expectations. The GEMV
expectation uses x = 1 for every element, or a ramp x[k] = k % 7 - 3, computed in
integer/exact arithmetic.

Run: python tests/golden/make_kat.py   (rewrites the JSON next to this file)
"""
from __future__ import annotations

import json
import struct
from fractions import Fraction
from pathlib import Path

HALF = {1.0: 0x3C00, 0.5: 0x3800, 0.25: 0x3400, 2.0: 0x4000, 0.125: 0x3000}


def h(v: float) -> bytes:
    return struct.pack("<H", HALF[v])


def q8_0_case():
    d = 0.5
    q = [((i * 37) % 255) - 127 for i in range(32)]
    blob = h(d) + bytes((v & 0xFF) for v in q)
    vals = [Fraction(d) * v for v in q]
    return "Q8_0", 8, 1, 32, blob, vals


def q4_0_case():
    blocks, vals = b"", []
    for blk, d in enumerate((1.0, 0.25)):
        q = [(3 * i + blk) % 16 for i in range(32)]  # element i's 4-bit code
        packed = bytes(q[i] | (q[i + 16] << 4) for i in range(16))  # lo nibble i, hi nibble i+16
        blocks += h(d) + packed
        vals += [Fraction(d) * (c - 8) for c in q]
    return "Q4_0", 2, 1, 64, blocks, vals


def q2_0_case():
    d = 2.0
    q = [(i * 5 + 1) % 4 for i in range(128)]
    packed = bytes(q[4 * p] | (q[4 * p + 1] << 2) | (q[4 * p + 2] << 4) | (q[4 * p + 3] << 6) for p in range(32))
    return "Q2_0", 42, 1, 128, h(d) + packed, [Fraction(d) * (c - 1) for c in q]


def q4_k_case():
    d, dmin = 1.0, 0.5
    sc = [1, 2, 3, 4, 33, 45, 58, 63]  # j >= 4 use the 2 high bits
    mn = [0, 5, 17, 31, 32, 48, 1, 63]
    s = [0] * 12
    for j in range(4):  # the 12-byte packing that get_scale_min_k4 decodes
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    code = [(7 * e + e // 32) % 16 for e in range(256)]
    qs = bytearray(128)
    for c in range(4):  # 32-byte group c: lo nibble -> element 64c+l, hi -> 64c+32+l
        for l in range(32):
            qs[32 * c + l] = code[64 * c + l] | (code[64 * c + 32 + l] << 4)
    blob = h(d) + h(dmin) + bytes(s) + bytes(qs)
    vals = [Fraction(d) * sc[e // 32] * code[e] - Fraction(dmin) * mn[e // 32] for e in range(256)]
    return "Q4_K", 12, 1, 256, blob, vals


def q6_k_case():
    d = 0.25
    sc = [1, -2, 3, -4, 5, -6, 7, -8, 127, -127, 64, -64, 9, -10, 11, -12]
    code = [(11 * e + 3) % 64 for e in range(256)]
    ql, qh = bytearray(128), bytearray(64)
    for half in range(2):  # 128-element halves: ql += 64, qh += 32
        for l in range(32):
            e = 128 * half
            q1, q2, q3, q4 = code[e + l], code[e + l + 32], code[e + l + 64], code[e + l + 96]
            ql[64 * half + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[64 * half + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            qh[32 * half + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    blob = bytes(ql) + bytes(qh) + bytes((v & 0xFF) for v in sc) + h(d)
    # (d*sc)*q in IEEE arithmetic: a zero code under a negative scale is -0.0
    vals = [Fraction(d) * sc[e // 16] * (code[e] - 32) if code[e] != 32 else (-0.0 if sc[e // 16] < 0 else 0.0)
            for e in range(256)]
    return "Q6_K", 14, 1, 256, blob, vals


def main() -> None:
    cases = []
    for fn in (q8_0_case, q4_0_case, q2_0_case, q4_k_case, q6_k_case):
        name, tid, rows, cols, blob, vals = fn()
        ones = sum(vals)
        ramp = sum(v * ((k % 7) - 3) for k, v in enumerate(vals))
        cases.append(
            {
                "name": name,
                "type_id": tid,
                "rows": rows,
                "cols": cols,
                "blob_hex": blob.hex(),
                "values": [v if isinstance(v, float) else float(v) for v in vals],
                "gemv_x_ones": float(ones),
                "gemv_x_ramp": float(ramp),
            }
        )
    out = Path(__file__).with_name("kat_blocks.json")
    out.write_text(json.dumps({"cases": cases}, indent=1) + "\n")
    print(f"wrote {out} ({len(cases)} cases)")


if __name__ == "__main__":
    main()

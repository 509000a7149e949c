// Seeded synthetic GGUF blocks and activations, bit-identical on host and device.
//
// Counter-based: every random draw is mix64(seed + 0x9E3779B97F4A7C15 * counter), the
// SplitMix64 finaliser the reference uses for its own counter-based generators
// (jax4j-core/.../tensor/spi/ComputeBackend.java:282-295). Uniform floats take the top 24
// bits; normals use Box-Muller in double as the reference's randomNormal does
// (ComputeBackend.java:63-76). Each value has its own counter, so any block can be
// produced independently by any thread. Distributions follow the benchmark configs:
//   Q8_0: d = fp16(|N(0,1)|*0.02), q ~ U{-127..127}
//   Q4_0: d = fp16(|N(0,1)|*0.05), q ~ U{0..15}
//   Q4_K: d = fp16(|N|*0.002), dmin = fp16(|N|*0.001), scales/mins ~ U{0..63}, q ~ U{0..15}
//   Q6_K: d = fp16(|N|*0.001), scales = clip(round(N(0,20)), -127, 127), q ~ U{0..63}
//   Q2_0: d = fp16(|N|*0.05), q ~ U{0..3}
//   x   : N(0,1) fp32; bf16 activations are the RNE bf16 of N(0,1)
#pragma once

#include <math.h>
#include <stdint.h>

#ifdef __HIPCC__
#define J4Q_HD __host__ __device__ __forceinline__
#else
#define J4Q_HD static inline
#endif

namespace j4q_synth {

enum Stream : uint64_t { S_SCALE = 1, S_SCALE2 = 2, S_SUB = 3, S_QUANT = 4, S_X = 5 };

J4Q_HD uint64_t mix64(uint64_t v) {
    v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
    v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
    return v ^ (v >> 31);
}

J4Q_HD uint64_t draw(uint64_t seed, uint64_t stream, uint64_t index) {
    return mix64(seed + 0x9E3779B97F4A7C15ull * ((stream << 56) ^ index));
}

// Uniform integer in [0, n) from the top 24 bits.
J4Q_HD uint32_t uniform_int(uint64_t seed, uint64_t stream, uint64_t index, uint32_t n) {
    return (uint32_t)(((draw(seed, stream, index) >> 40) * (uint64_t)n) >> 24);
}

J4Q_HD double normal(uint64_t seed, uint64_t stream, uint64_t index) {
    const double u1 = (double)((draw(seed, stream, 2 * index) >> 40) + 1) * 0x1.0p-24;
    const double u2 = (double)(draw(seed, stream, 2 * index + 1) >> 40) * 0x1.0p-24;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

J4Q_HD uint32_t f32_bits(float f) {
    union {
        float f;
        uint32_t u;
    } c;
    c.f = f;
    return c.u;
}

J4Q_HD float bits_f32(uint32_t u) {
    union {
        float f;
        uint32_t u;
    } c;
    c.u = u;
    return c.f;
}

// fp32 -> fp16, round to nearest even, integer-only so host and device agree exactly.
J4Q_HD uint16_t f32_to_f16(float f) {
    const uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520: inf
    if (ax < 0x33000001u) return (uint16_t)sign;                // |f| <= 2^-25: zero
    const int e = (int)(ax >> 23);
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    int shift;
    uint32_t base;
    if (e < 113) {  // fp16 subnormal
        shift = 126 - e;
        base = 0;
    } else {
        shift = 13;
        base = (uint32_t)(e - 112) << 10;
        mant &= 0x7fffffu;
    }
    const uint32_t half_ulp = 1u << (shift - 1);
    const uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t r = (mant >> shift);
    if (rem > half_ulp || (rem == half_ulp && (r & 1u))) r += 1;
    return (uint16_t)(sign | (base + r));
}

// fp32 -> bf16, round to nearest even (NaN stays quiet).
J4Q_HD uint16_t f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

J4Q_HD uint16_t abs_normal_scale_f16(uint64_t seed, uint64_t stream, uint64_t index, double mul) {
    return f32_to_f16((float)(fabs(normal(seed, stream, index)) * mul));
}

J4Q_HD void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}

// Writes GGUF block `bi` (row-major block index) of a matrix with `cols` columns.
// Returns the number of bytes written, 0 for an unknown type id.
J4Q_HD int synth_block(int id, uint64_t seed, uint64_t bi, int64_t cols, uint8_t *out) {
    switch (id) {
    case 8: {  // Q8_0
        const uint64_t bpr = (uint64_t)cols / 32, row = bi / bpr, e0 = row * (uint64_t)cols + (bi % bpr) * 32;
        put16(out, abs_normal_scale_f16(seed, S_SCALE, bi, 0.02));
        for (int i = 0; i < 32; i++) out[2 + i] = (uint8_t)(int8_t)((int)uniform_int(seed, S_QUANT, e0 + i, 255) - 127);
        return 34;
    }
    case 2: {  // Q4_0
        const uint64_t bpr = (uint64_t)cols / 32, row = bi / bpr, e0 = row * (uint64_t)cols + (bi % bpr) * 32;
        put16(out, abs_normal_scale_f16(seed, S_SCALE, bi, 0.05));
        for (int i = 0; i < 16; i++) {
            const uint32_t lo = uniform_int(seed, S_QUANT, e0 + i, 16);
            const uint32_t hi = uniform_int(seed, S_QUANT, e0 + 16 + i, 16);
            out[2 + i] = (uint8_t)(lo | (hi << 4));
        }
        return 18;
    }
    case 12: {  // Q4_K
        const uint64_t bpr = (uint64_t)cols / 256, row = bi / bpr, e0 = row * (uint64_t)cols + (bi % bpr) * 256;
        put16(out, abs_normal_scale_f16(seed, S_SCALE, bi, 0.002));
        put16(out + 2, abs_normal_scale_f16(seed, S_SCALE2, bi, 0.001));
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)uniform_int(seed, S_SUB, bi * 16 + j, 64);
            mn[j] = (uint8_t)uniform_int(seed, S_SUB, bi * 16 + 8 + j, 64);
        }
        uint8_t *s = out + 4;  // ggml 12-byte packing (inverse of get_scale_min_k4)
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
        }
        uint8_t *q = out + 16;  // 32-byte group c: lo nibble elem 64c+l, hi nibble 64c+32+l
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                const uint32_t lo = uniform_int(seed, S_QUANT, e0 + 64 * c + l, 16);
                const uint32_t hi = uniform_int(seed, S_QUANT, e0 + 64 * c + 32 + l, 16);
                q[32 * c + l] = (uint8_t)(lo | (hi << 4));
            }
        return 144;
    }
    case 14: {  // Q6_K
        const uint64_t bpr = (uint64_t)cols / 256, row = bi / bpr, e0 = row * (uint64_t)cols + (bi % bpr) * 256;
        uint8_t *ql = out, *qh = out + 128;
        for (int i = 0; i < 64; i++) qh[i] = 0;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                uint32_t q[4];
                for (int t = 0; t < 4; t++) q[t] = uniform_int(seed, S_QUANT, e0 + 128 * h + 32 * t + l, 64);
                ql[64 * h + l] = (uint8_t)((q[0] & 15) | ((q[2] & 15) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((q[1] & 15) | ((q[3] & 15) << 4));
                qh[32 * h + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
            }
        for (int j = 0; j < 16; j++) {
            double v = nearbyint(normal(seed, S_SUB, bi * 16 + j) * 20.0);
            if (v > 127.0) v = 127.0;
            if (v < -127.0) v = -127.0;
            out[192 + j] = (uint8_t)(int8_t)(int)v;
        }
        put16(out + 208, abs_normal_scale_f16(seed, S_SCALE, bi, 0.001));
        return 210;
    }
    case 42: {  // Q2_0
        const uint64_t bpr = (uint64_t)cols / 128, row = bi / bpr, e0 = row * (uint64_t)cols + (bi % bpr) * 128;
        put16(out, abs_normal_scale_f16(seed, S_SCALE, bi, 0.05));
        for (int p = 0; p < 32; p++) {
            uint32_t v = 0;
            for (int s = 0; s < 4; s++) v |= uniform_int(seed, S_QUANT, e0 + 4 * p + s, 4) << (2 * s);
            out[2 + p] = (uint8_t)v;
        }
        return 34;
    }
    default: return 0;
    }
}

J4Q_HD float synth_x(uint64_t seed, uint64_t i) { return (float)normal(seed, S_X, i); }

}  // namespace j4q_synth

// Prefill GEMM over Q8_0 weights: activation quantizer and the two MFMA variants.
#include "j4q_common.h"

namespace j4q {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// One thread per (row, 32-element block): s = amax/127, q = clamp(roundf(x * (1/s)), +-127)
// (ggml quantize_row_q8_0 with the scale kept in fp32). Division and the reciprocal are
// IEEE correctly rounded, so the result is bit-identical to a C reference.
__global__ void __launch_bounds__(256)
quantize_act_kernel(const uint16_t *__restrict__ x, int64_t m, int64_t k, int8_t *__restrict__ q, float *__restrict__ s) {
    const int64_t nb = k / 32;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= m * nb) return;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(x + t * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u32x4 p = src[i];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[8 * i + 2 * j] = __builtin_bit_cast(float, p[j] << 16);
            v[8 * i + 2 * j + 1] = __builtin_bit_cast(float, p[j] & 0xffff0000u);
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    u32x4 out[2];
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float r = __builtin_roundf(v[i] * id);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        const uint32_t b = (uint32_t)(uint8_t)(int8_t)(int)r;
        if ((i & 3) == 0) out[i >> 4][(i >> 2) & 3] = 0;
        out[i >> 4][(i >> 2) & 3] |= b << (8 * (i & 3));
    }
    u32x4 *dst = reinterpret_cast<u32x4 *>(q + t * 32);
    dst[0] = out[0];
    dst[1] = out[1];
    s[t] = d;
}

}  // namespace

hipError_t launch_quantize_act(const uint16_t *x, int64_t m, int64_t k, int8_t *q, float *scales, hipStream_t s) {
    const int64_t n = m * (k / 32);
    if (n == 0) return hipSuccess;
    quantize_act_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, m, k, q, scales);
    return hipGetLastError();
}

hipError_t launch_gemm_q8_int8(const QMat &, const int8_t *, const float *, float *, int64_t, hipStream_t) {
    return hipErrorNotSupported;
}

hipError_t launch_gemm_q8_bf16(const QMat &, const uint16_t *, float *, int64_t, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace j4q

/*
 * CPU oracle for the GGUF block-quantized matmul path -- TEST INFRASTRUCTURE ONLY.
 * See quant_ref.h for the rules on who may load this code and for the citation prefixes.
 *
 * Built with -O2 -ffp-contract=off and no fast-math, so every float '*' and '+' below
 * rounds exactly once, as Java's strict float arithmetic does in the reference loops.
 */
#include "quant_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t float_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

int ref_block_geometry(int type_id, int *block_elements, int *block_bytes) {
    /* tensor/QuantType.java:5-13 (only the block-quantized rows this path handles). */
    int be, bb;
    switch (type_id) {
    case REF_Q4_0: be = 32; bb = 18; break;
    case REF_Q8_0: be = 32; bb = 34; break;
    case REF_Q4_K: be = 256; bb = 144; break;
    case REF_Q6_K: be = 256; bb = 210; break;
    case REF_Q2_0: be = 128; bb = 34; break;
    default: return -1;
    }
    if (block_elements) *block_elements = be;
    if (block_bytes) *block_bytes = bb;
    return 0;
}

/* cpu/CpuQ4Gemm.java:58-77: subnormals are normalised by shifting the fraction up
 * while decrementing the exponent; Inf/NaN keep the payload shifted by 13. */
float ref_half_to_float(uint32_t bits) {
    uint32_t sign = (bits & 0x8000u) << 16;
    int32_t exponent = (int32_t)((bits >> 10) & 0x1f);
    uint32_t fraction = bits & 0x3ffu;
    if (exponent == 0) {
        if (fraction == 0) return bits_to_float(sign);
        exponent = 1;
        while ((fraction & 0x400u) == 0) {
            fraction <<= 1;
            exponent--;
        }
        return bits_to_float(sign | ((uint32_t)(exponent + 112) << 23) | ((fraction & 0x3ffu) << 13));
    }
    if (exponent == 31) return bits_to_float(sign | 0x7f800000u | (fraction << 13));
    return bits_to_float(sign | ((uint32_t)(exponent + 112) << 23) | (fraction << 13));
}

void ref_half_to_float_array(const uint16_t *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = ref_half_to_float(in[i]);
}

static float half_at(const uint8_t *p) { return ref_half_to_float((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

/* cpu/CpuQ4Gemm.java:79-83 (validate). */
static int valid_dims(int64_t rows, int64_t cols, int64_t block) {
    return rows > 0 && cols > 0 && cols % block == 0;
}

/* cpu/CpuQ4Gemm.java:26-46. One float accumulator per row; within each 32-element block
 * the 16 packed bytes are visited in order, low nibble (element p) then high nibble
 * (element p+16); each term is (scale*(q-8))*x rounded, then added. */
int ref_q4_0_multiply(float *out, const float *input, const uint8_t *weights, int64_t rows, int64_t cols) {
    if (!valid_dims(rows, cols, 32)) return -1;
    const int64_t blocks = cols / 32;
    for (int64_t row = 0; row < rows; row++) {
        float sum = 0.0f;
        const int64_t row_offset = row * blocks * 18;
        for (int64_t block = 0; block < blocks; block++) {
            const uint8_t *b = weights + row_offset + block * 18;
            const float scale = half_at(b);
            const int64_t base = block * 32;
            for (int p = 0; p < 16; p++) {
                const int packed = b[2 + p];
                const int low = packed & 0x0f;
                const int high = (packed >> 4) & 0x0f;
                float t = scale * (float)(low - 8);
                t = t * input[base + p];
                sum = sum + t;
                t = scale * (float)(high - 8);
                t = t * input[base + p + 16];
                sum = sum + t;
            }
        }
        out[row] = sum;
    }
    return 0;
}

/* cpu/CpuQ4Gemm.java:48-56 (packedValue). */
static float q4_0_packed_value(const uint8_t *weights, int64_t row_offset, int64_t index) {
    const int64_t block = index / 32;
    const int within = (int)(index % 32);
    const uint8_t *b = weights + row_offset + block * 18;
    const float scale = half_at(b);
    const int packed = b[2 + (within % 16)];
    const int nibble = within < 16 ? (packed & 0x0f) : ((packed >> 4) & 0x0f);
    return scale * (float)(nibble - 8);
}

/* cpu/CpuQ4Gemm.java:17-24. The reference does not range-check `row`; reading past the
 * array throws in Java, which this restatement reports as -1. */
int ref_q4_0_gather(float *out, const uint8_t *weights, int64_t row, int64_t rows, int64_t cols) {
    if (!valid_dims(rows, cols, 32)) return -1;
    if (row < 0 || row >= rows) return -1;
    const int64_t row_bytes = cols / 32 * 18;
    for (int64_t i = 0; i < cols; i++) out[i] = q4_0_packed_value(weights, row * row_bytes, i);
    return 0;
}

/* cpu/CpuQ2Gemm.java:26-46: 128 elements / 34 bytes, value = scale*(2-bit - 1), four
 * elements per byte in ascending bit order. */
int ref_q2_0_multiply(float *out, const float *input, const uint8_t *weights, int64_t rows, int64_t cols) {
    if (!valid_dims(rows, cols, 128)) return -1;
    const int64_t blocks = cols / 128;
    for (int64_t row = 0; row < rows; row++) {
        float sum = 0.0f;
        const int64_t row_offset = row * blocks * 34;
        for (int64_t block = 0; block < blocks; block++) {
            const uint8_t *b = weights + row_offset + block * 34;
            const float scale = half_at(b);
            const int64_t base = block * 128;
            for (int p = 0; p < 32; p++) {
                const int packed = b[2 + p];
                const int64_t index = base + ((int64_t)p << 2);
                for (int s = 0; s < 4; s++) {
                    float t = scale * (float)(((packed >> (2 * s)) & 3) - 1);
                    t = t * input[index + s];
                    sum = sum + t;
                }
            }
        }
        out[row] = sum;
    }
    return 0;
}

/* cpu/CpuQ2Gemm.java:17-24, 49-56. */
int ref_q2_0_gather(float *out, const uint8_t *weights, int64_t row, int64_t rows, int64_t cols) {
    if (!valid_dims(rows, cols, 128)) return -1;
    if (row < 0 || row >= rows) return -1;
    const int64_t row_offset = row * (cols / 128 * 34);
    for (int64_t i = 0; i < cols; i++) {
        const uint8_t *b = weights + row_offset + (i / 128) * 34;
        const int within = (int)(i % 128);
        const float scale = half_at(b);
        const int packed = b[2 + within / 4];
        out[i] = scale * (float)(((packed >> ((within & 3) * 2)) & 3) - 1);
    }
    return 0;
}

/* ggml dequantize_row_q8_0: y = d * qs[i]. */
static void dq_q8_0(const uint8_t *b, float *y) {
    const float d = half_at(b);
    for (int i = 0; i < 32; i++) y[i] = d * (float)(int8_t)b[2 + i];
}

/* ggml get_scale_min_k4: 6-bit sub-block scale and min out of the 12 packed bytes. */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* ggml dequantize_row_q4_K: 144-byte superblock [d | dmin | scales[12] | qs[128]];
 * 64-element chunk c uses qs[32c..32c+32): low nibbles -> sub-block 2c, high -> 2c+1;
 * y = (d*sc)*q - (dmin*m). */
static void dq_q4_k(const uint8_t *b, float *y) {
    const float d = half_at(b);
    const float dmin = half_at(b + 2);
    const uint8_t *scales = b + 4;
    const uint8_t *q = b + 16;
    int is = 0;
    for (int j = 0; j < 256; j += 64) {
        int sc, m;
        scale_min_k4(is + 0, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; l++) y[j + l] = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) y[j + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        q += 32;
        is += 2;
    }
}

/* ggml dequantize_row_q6_K: 210-byte superblock [ql[128] | qh[64] | scales int8[16] | d];
 * per 128-element half: ql advances 64, qh 32, scales 8. */
static void dq_q6_k(const uint8_t *b, float *y) {
    const float d = half_at(b + 208);
    const uint8_t *ql = b;
    const uint8_t *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[n + l + 0] = d * (float)sc[is + 0] * (float)q1;
            y[n + l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[n + l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[n + l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

int ref_dequant_row(int type_id, const uint8_t *row_blocks, int64_t cols, float *out) {
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0 || cols <= 0 || cols % be != 0) return -1;
    const int64_t nb = cols / be;
    switch (type_id) {
    case REF_Q4_0: return ref_q4_0_gather(out, row_blocks, 0, 1, cols);
    case REF_Q2_0: return ref_q2_0_gather(out, row_blocks, 0, 1, cols);
    case REF_Q8_0:
        for (int64_t i = 0; i < nb; i++) dq_q8_0(row_blocks + i * bb, out + i * be);
        return 0;
    case REF_Q4_K:
        for (int64_t i = 0; i < nb; i++) dq_q4_k(row_blocks + i * bb, out + i * be);
        return 0;
    case REF_Q6_K:
        for (int64_t i = 0; i < nb; i++) dq_q6_k(row_blocks + i * bb, out + i * be);
        return 0;
    default: return -1;
    }
}

static int64_t row_bytes_of(int type_id, int64_t cols) {
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0) return -1;
    return cols / be * bb;
}

int ref_matvec(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, const float *x, float *y) {
    if (type_id == REF_Q4_0) return ref_q4_0_multiply(y, x, blob, rows, cols);
    if (type_id == REF_Q2_0) return ref_q2_0_multiply(y, x, blob, rows, cols);
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0 || !valid_dims(rows, cols, be)) return -1;
    float *w = (float *)malloc((size_t)cols * sizeof(float));
    if (!w) return -1;
    const int64_t rb = row_bytes_of(type_id, cols);
    for (int64_t r = 0; r < rows; r++) {
        ref_dequant_row(type_id, blob + r * rb, cols, w);
        float sum = 0.0f;
        for (int64_t k = 0; k < cols; k++) {
            const float t = w[k] * x[k];
            sum = sum + t;
        }
        y[r] = sum;
    }
    free(w);
    return 0;
}

int ref_matvec_f64(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, const float *x, double *y) {
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0 || !valid_dims(rows, cols, be)) return -1;
    float *w = (float *)malloc((size_t)cols * sizeof(float));
    if (!w) return -1;
    const int64_t rb = row_bytes_of(type_id, cols);
    for (int64_t r = 0; r < rows; r++) {
        ref_dequant_row(type_id, blob + r * rb, cols, w);
        double sum = 0.0;
        for (int64_t k = 0; k < cols; k++) sum += (double)w[k] * (double)x[k];
        y[r] = sum;
    }
    free(w);
    return 0;
}

/* ref_matvec_f64 for a batch of B activation rows x[B][cols] -> y[B][rows]: each weight row
 * is decoded once and dotted with every batch row in the same order as ref_matvec_f64, so
 * row b equals ref_matvec_f64 of x[b] exactly (semantics: CpuBackend.java:708-725 per row). */
int ref_matmul_f64(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, const float *x, int64_t batch,
                   double *y) {
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0 || !valid_dims(rows, cols, be) || batch <= 0) return -1;
    float *w = (float *)malloc((size_t)cols * sizeof(float));
    if (!w) return -1;
    const int64_t rb = row_bytes_of(type_id, cols);
    for (int64_t r = 0; r < rows; r++) {
        ref_dequant_row(type_id, blob + r * rb, cols, w);
        for (int64_t b = 0; b < batch; b++) {
            const float *xb = x + b * cols;
            double sum = 0.0;
            for (int64_t k = 0; k < cols; k++) sum += (double)w[k] * (double)xb[k];
            y[b * rows + r] = sum;
        }
    }
    free(w);
    return 0;
}

int ref_dequant_matrix(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, float *out) {
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0 || !valid_dims(rows, cols, be)) return -1;
    const int64_t rb = row_bytes_of(type_id, cols);
    for (int64_t r = 0; r < rows; r++) ref_dequant_row(type_id, blob + r * rb, cols, out + r * cols);
    return 0;
}

uint16_t ref_f32_to_bf16(float f) {
    uint32_t u = float_to_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float ref_bf16_to_f32(uint16_t h) { return bits_to_float((uint32_t)h << 16); }

int ref_quantize_act(const uint16_t *x_bf16, int64_t m, int64_t k, int8_t *q, float *scales) {
    if (m <= 0 || k <= 0 || k % 32 != 0) return -1;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < m; i++) {
        for (int64_t b = 0; b < nb; b++) {
            const uint16_t *xb = x_bf16 + i * k + b * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) {
                const float v = fabsf(ref_bf16_to_f32(xb[j]));
                if (v > amax) amax = v;
            }
            const float s = amax / 127.0f;
            const float id = s != 0.0f ? 1.0f / s : 0.0f;
            for (int j = 0; j < 32; j++) {
                float r = roundf(ref_bf16_to_f32(xb[j]) * id);
                if (r > 127.0f) r = 127.0f;
                if (r < -127.0f) r = -127.0f;
                q[i * k + b * 32 + j] = (int8_t)r;
            }
            scales[i * nb + b] = s;
        }
    }
    return 0;
}

int ref_gemm_q8_int8_emulated_ranges(const int8_t *xq, const float *xs, const uint8_t *w_blob, int64_t m,
                                     int64_t n, int64_t k, int64_t nranges, int64_t stage_blocks, float *y) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 32 != 0 || nranges < 1 || nranges > 8 || stage_blocks < 1) return -1;
    const int64_t nb = k / 32;
    const int64_t stages = (nb + stage_blocks - 1) / stage_blocks;
    const int64_t span = (stages + nranges - 1) / nranges * stage_blocks; /* blocks per range */
    for (int64_t i = 0; i < m; i++) {
        for (int64_t j = 0; j < n; j++) {
            float part[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t *wb = w_blob + (j * nb + b) * 34;
                const int8_t *xb = xq + i * k + b * 32;
                int32_t dot = 0;
                for (int t = 0; t < 32; t++) dot += (int32_t)xb[t] * (int32_t)(int8_t)wb[2 + t];
                const float s = xs[i * nb + b] * half_at(wb);
                part[b / span] = fmaf((float)dot, s, part[b / span]);
            }
            float acc = part[0];
            for (int64_t p = 1; p < nranges; p++) acc = acc + part[p];
            y[i * n + j] = acc;
        }
    }
    return 0;
}

int ref_gemm_q8_int8_emulated(const int8_t *xq, const float *xs, const uint8_t *w_blob, int64_t m, int64_t n,
                              int64_t k, float *y) {
    return ref_gemm_q8_int8_emulated_ranges(xq, xs, w_blob, m, n, k, 1, 1, y);
}

static int gemm_f64(int type_id, const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                    double *y, int round_w_to_bf16) {
    int be, bb;
    if (ref_block_geometry(type_id, &be, &bb) != 0 || m <= 0 || !valid_dims(n, k, be)) return -1;
    float *w = (float *)malloc((size_t)k * sizeof(float));
    double *xd = (double *)malloc((size_t)(m * k) * sizeof(double));
    if (!w || !xd) {
        free(w);
        free(xd);
        return -1;
    }
    for (int64_t t = 0; t < m * k; t++) xd[t] = (double)ref_bf16_to_f32(x_bf16[t]);
    const int64_t rb = row_bytes_of(type_id, k);
    for (int64_t j = 0; j < n; j++) {
        ref_dequant_row(type_id, w_blob + j * rb, k, w);
        if (round_w_to_bf16)
            for (int64_t t = 0; t < k; t++) w[t] = ref_bf16_to_f32(ref_f32_to_bf16(w[t]));
        for (int64_t i = 0; i < m; i++) {
            double s = 0.0;
            const double *xr = xd + i * k;
            for (int64_t t = 0; t < k; t++) s += xr[t] * (double)w[t];
            y[i * n + j] = s;
        }
    }
    free(w);
    free(xd);
    return 0;
}

int ref_gemm_f64(int type_id, const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                 double *y) {
    return gemm_f64(type_id, x_bf16, w_blob, m, n, k, y, 0);
}

int ref_gemm_bf16w_f64(int type_id, const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                       double *y) {
    return gemm_f64(type_id, x_bf16, w_blob, m, n, k, y, 1);
}

int ref_gemm_q8_f64(const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k, double *y) {
    return gemm_f64(REF_Q8_0, x_bf16, w_blob, m, n, k, y, 0);
}

int ref_gemm_q8_bf16w_f64(const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                          double *y) {
    return gemm_f64(REF_Q8_0, x_bf16, w_blob, m, n, k, y, 1);
}

/*
 * CPU oracle for the GGUF block-quantized matmul path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or the timed CPU baseline). The product path
 * (jax4j_amd/) never links or calls it.
 *
 * Every function cites the reference file:line it restates. Paths are relative to the
 * jax4j 0.2.1 checkout; `cpu/` = jax4j-core/src/main/java/com/nablatensor/jax4j/backend/cpu/.
 * Q8_0, Q4_K and Q6_K have no arithmetic in the reference (enum rows only,
 * tensor/QuantType.java:8-10; rejected at cpu/CpuBackend.java:698-701): those functions
 * restate the public ggml block formats (ggml-common.h block structs, ggml-quants.c
 * dequantize_row_* / quantize_row_q8_0; not vendored by the reference, no pinned version).
 */
#ifndef JAX4J_ORACLE_QUANT_REF_H
#define JAX4J_ORACLE_QUANT_REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (tensor/QuantType.java:5-13). */
enum { REF_Q4_0 = 2, REF_Q8_0 = 8, REF_Q4_K = 12, REF_Q6_K = 14, REF_Q2_0 = 42 };

/* Status: 0 ok, -1 invalid dimensions / unsupported type (IllegalArgumentException). */

/* Block geometry (tensor/QuantType.java:5-13). Returns -1 for unknown ids. */
int ref_block_geometry(int type_id, int *block_elements, int *block_bytes);

/* IEEE binary16 -> binary32 (cpu/CpuQ4Gemm.java:58-77). */
float ref_half_to_float(uint32_t bits);
/* Same over an array (keeps signaling-NaN payloads intact for bitwise comparison). */
void ref_half_to_float_array(const uint16_t *in, float *out, int64_t n);

/* Q4_0 fused dequant GEMV, sequential float accumulator (cpu/CpuQ4Gemm.java:26-46). */
int ref_q4_0_multiply(float *out, const float *input, const uint8_t *weights, int64_t rows, int64_t cols);
/* Q4_0 row gather (cpu/CpuQ4Gemm.java:17-24, 48-56). */
int ref_q4_0_gather(float *out, const uint8_t *weights, int64_t row, int64_t rows, int64_t cols);
/* Q2_0 (prism fork) GEMV and gather (cpu/CpuQ2Gemm.java:26-46, 17-24, 49-56). */
int ref_q2_0_multiply(float *out, const float *input, const uint8_t *weights, int64_t rows, int64_t cols);
int ref_q2_0_gather(float *out, const uint8_t *weights, int64_t row, int64_t rows, int64_t cols);

/* Dequantize one row of any supported type to fp32 (Q4_0/Q2_0: the reference's gather;
 * Q8_0/Q4_K/Q6_K: ggml dequantize_row_*). `row_blocks` points at the row's first block. */
int ref_dequant_row(int type_id, const uint8_t *row_blocks, int64_t cols, float *out);

/* y[r] = sum_k W[r,k] x[k], float accumulator in natural element order over the ggml
 * dequantized values (the "restated ggml scalar loop"); Q4_0/Q2_0 use the reference's
 * own loop order instead (cpu/CpuQ4Gemm.java:26-46). */
int ref_matvec(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, const float *x, float *y);
/* Same product accumulated in double: the brute-force tolerance reference. */
int ref_matvec_f64(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, const float *x, double *y);
/* ref_matvec_f64 over a batch: x [batch][cols] -> y [batch][rows]; row b equals
 * ref_matvec_f64 of x[b] bit for bit (one decode of each weight row). */
int ref_matmul_f64(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, const float *x, int64_t batch,
                   double *y);
/* Full-matrix dequantization, rows x cols fp32. */
int ref_dequant_matrix(int type_id, const uint8_t *blob, int64_t rows, int64_t cols, float *out);

/* bf16 helpers: round-to-nearest-even fp32 -> bf16, and bf16 -> fp32. */
uint16_t ref_f32_to_bf16(float f);
float ref_bf16_to_f32(uint16_t h);

/* Activation quantizer for the prefill GEMM: per row, per 32-element block,
 * amax = max|x|, s = amax/127, id = s ? 1/s : 0, q = clamp(roundf(x*id), -127, 127).
 * Mirrors ggml quantize_row_q8_0 with the scale kept in fp32. x is bf16 [m, k]. */
int ref_quantize_act(const uint16_t *x_bf16, int64_t m, int64_t k, int8_t *q, float *scales);

/* Emulated int8 GEMM: for each block b in order, acc = fmaf((float)dot_b, sx[i,b]*dw[j,b], acc)
 * with dot_b = sum_{k in b} qx*qw exact in int32 and the scale product rounded to fp32.
 * W is Q8_0 [n, k]. The tight (bit-exact) check for the int8 path. */
int ref_gemm_q8_int8_emulated(const int8_t *xq, const float *xs, const uint8_t *w_blob,
                              int64_t m, int64_t n, int64_t k, float *y);
/* The same with K cut into nranges contiguous ranges of whole stages (stage_blocks blocks
 * each; every range but the last ceil(stages / nranges) stages): each range folds its blocks
 * in order into its own partial from 0, then y = ((p0 + p1) + p2) + ... (nranges = 1: the
 * above). The GPU's small-M int8 kernel uses four ranges of four-block stages. */
int ref_gemm_q8_int8_emulated_ranges(const int8_t *xq, const float *xs, const uint8_t *w_blob, int64_t m,
                                     int64_t n, int64_t k, int64_t nranges, int64_t stage_blocks, float *y);
/* Exact reference for both GEMM variants: Y = X_bf16 . dequant(W)^T in double, W of any
 * supported type [n, k] (semantics: quantMatvec per row of X, cpu/CpuBackend.java:708-725,
 * over the exactly decoded weights of ref_dequant_row). */
int ref_gemm_f64(int type_id, const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                 double *y);
/* bf16 variant emulation: Y = X_bf16 . bf16(dequant(W))^T in double (every fp32 weight of
 * ref_dequant_row rounded to the nearest-even bf16 first). */
int ref_gemm_bf16w_f64(int type_id, const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                       double *y);
/* The two above for Q8_0 weights. */
int ref_gemm_q8_f64(const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k, double *y);
int ref_gemm_q8_bf16w_f64(const uint16_t *x_bf16, const uint8_t *w_blob, int64_t m, int64_t n, int64_t k,
                          double *y);

#ifdef __cplusplus
}
#endif
#endif

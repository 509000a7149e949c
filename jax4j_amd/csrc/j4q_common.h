// Shared definitions for the MI355X (gfx950) GGUF quantized-matmul engine.
//
// Engine-resident weight layout ("split layout"). uploadQuantized copies the caller's
// GGUF blob to HBM and repacks it once into per-row arrays whose 16-byte chunks each
// hold 32 consecutive elements, so the GEMV streams every row with aligned 128-bit
// loads. The repack is a bijection on bits: gather/export reproduce the GGUF values bit
// for bit, and bytes per matrix are the GGUF byte count (plus, for Q8_0 only, a second
// copy of the scales for the prefill GEMM).
//
//   Q4_0 : qs  [N][K/2]    chunk j byte i: lo nibble = elem 32j+i, hi = elem 32j+16+i
//          sc  [N][K/32]   fp16 d
//   Q8_0 : qs  [N][K]      int8, natural order
//          sc  [N][K/32]   fp16 d
//          d   [K/32][N]   the same fp16 d block-major: the 16 rows of a GEMM operand
//                          tile read one cache line per block
//   Q4_K : qs  [N][K/2]    chunk = one 32-element sub-block, nibble order as Q4_0
//          sc  [N][K/256]  16 B: d fp16 | dmin fp16 | D0 | D1 | D2 where
//                          D0 nibble j = scale_j & 15, D1 nibble j = min_j & 15,
//                          D2 bits 2j..2j+1 = scale_j >> 4, bits 16+2j.. = min_j >> 4
//   Q6_K : qs  [N][K/2]    low 4 bits, nibble order as Q4_0
//          qh  [N][K/4]    high 2 bits, two dwords per 32-element chunk (see gemv.hip)
//          sc  [N][K/16]   int8 group scales
//          d   [N][K/256]  fp16 d
//   Q2_0 : qs  [N][K/4]    GGUF order (byte p holds elements 4p..4p+3, 2 bits each)
//          sc  [N][K/128]  fp16 d
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace j4q {

enum QuantId : int { Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q6_K = 14, Q2_0 = 42 };

struct Geometry {
    int block_elements;
    int block_bytes;
};

// tensor/QuantType.java:5-13 (the block-quantized rows this engine accepts).
__host__ __device__ inline bool geometry_of(int id, Geometry *g) {
    switch (id) {
    case Q4_0: *g = {32, 18}; return true;
    case Q8_0: *g = {32, 34}; return true;
    case Q4_K: *g = {256, 144}; return true;
    case Q6_K: *g = {256, 210}; return true;
    case Q2_0: *g = {128, 34}; return true;
    default: return false;
    }
}

// Device view of one resident quantized matrix in the split layout above.
struct QMat {
    const uint8_t *qs;
    const uint8_t *qh;
    const uint8_t *sc;
    const uint8_t *d;
    int64_t rows;
    int64_t cols;
};

// Byte offsets of each section inside the single allocation that holds a matrix.
struct SplitLayout {
    uint64_t qs_off, qs_bytes;
    uint64_t qh_off, qh_bytes;
    uint64_t sc_off, sc_bytes;
    uint64_t d_off, d_bytes;
    uint64_t total;
};

__host__ __device__ inline uint64_t align256(uint64_t v) { return (v + 255u) & ~uint64_t(255); }

__host__ __device__ inline SplitLayout split_layout(int id, int64_t rows, int64_t cols) {
    SplitLayout L{};
    const uint64_t n = (uint64_t)rows, k = (uint64_t)cols;
    switch (id) {
    case Q4_0: L.qs_bytes = n * k / 2; L.sc_bytes = n * (k / 32) * 2; break;
    case Q8_0: L.qs_bytes = n * k; L.sc_bytes = n * (k / 32) * 2; L.d_bytes = L.sc_bytes; break;
    case Q4_K: L.qs_bytes = n * k / 2; L.sc_bytes = n * (k / 256) * 16; break;
    case Q6_K:
        L.qs_bytes = n * k / 2;
        L.qh_bytes = n * k / 4;
        L.sc_bytes = n * (k / 16);
        L.d_bytes = n * (k / 256) * 2;
        break;
    case Q2_0: L.qs_bytes = n * k / 4; L.sc_bytes = n * (k / 128) * 2; break;
    default: break;
    }
    uint64_t off = 0;
    L.qs_off = off; off = align256(off + L.qs_bytes);
    L.qh_off = off; off = align256(off + L.qh_bytes);
    L.sc_off = off; off = align256(off + L.sc_bytes);
    L.d_off = off; off = align256(off + L.d_bytes);
    L.total = off;
    return L;
}

__host__ __device__ inline QMat qmat_view(const uint8_t *base, int id, int64_t rows, int64_t cols) {
    const SplitLayout L = split_layout(id, rows, cols);
    QMat m;
    m.qs = base + L.qs_off;
    m.qh = L.qh_bytes ? base + L.qh_off : nullptr;
    m.sc = base + L.sc_off;
    m.d = L.d_bytes ? base + L.d_off : nullptr;
    m.rows = rows;
    m.cols = cols;
    return m;
}

// IEEE binary16 -> binary32; exact (the hardware conversion, v_cvt_f32_f16).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

}  // namespace j4q

// Kernel launchers implemented in the .hip translation units (host side).
namespace j4q {
hipError_t launch_repack(int id, const uint8_t *gguf, uint8_t *split, int64_t rows, int64_t cols,
                         hipStream_t s);
// Q8_0: rewrite the block-major scale copy (d) from the row-major scales (sc).
hipError_t launch_q8_scales_t(const QMat &m, hipStream_t s);
hipError_t launch_export(int id, const uint8_t *split, uint8_t *gguf, int64_t rows, int64_t cols,
                         hipStream_t s);
hipError_t launch_dequant_rows(int id, const QMat &m, int64_t row0, int64_t nrows, float *out,
                               hipStream_t s);
// Device scratch a batched GEMV may use for the partial sums of its column windows.
struct Workspace {
    float *ptr = nullptr;
    uint64_t bytes = 0;
};
// Bytes of workspace a batched GEMV of `batch` rows uses to run all its column windows in one
// launch (0 when it has one window, or does not run on the matrix cores). With less, the
// windows run one launch after another.
uint64_t gemv_workspace_bytes(int id, const QMat &m, int64_t batch);
// Whether an add that overlaps y is served for this matrix and batch (given the workspace
// gemv_workspace_bytes asks for): one column window, or the matrix-core path.
bool gemv_in_place_ok(int id, const QMat &m, int64_t batch);
// Batched GEMV arithmetic (J4Q_GEMV_MATRIX_CORES or J4Q_GEMV_FP32), process-wide; launches
// read it when they are issued.
void gemv_set_policy(int policy);
int gemv_policy();
hipError_t launch_gemv(int id, const QMat &m, const float *x, const float *add, float *y, int64_t batch,
                       hipStream_t s, const Workspace &ws = Workspace());
hipError_t launch_quantize_act(const uint16_t *x, int64_t m, int64_t k, int8_t *q, float *scales,
                               hipStream_t s);
hipError_t launch_gemm_q8_int8(const QMat &w, const int8_t *xq, const float *xs, float *y, int64_t m,
                               hipStream_t s);
hipError_t launch_gemm_q8_bf16(const QMat &w, const uint16_t *x, float *y, int64_t m, hipStream_t s);
// Prefill GEMM, bf16 variant, over Q4_0 (cols % 128 == 0), Q4_K and Q6_K weights.
bool gemm_kq_supported(int id, int64_t cols);
// Workspace the call needs (bytes; 0: none): the partial products of its K splits.
uint64_t gemm_kq_workspace_bytes(int id, const QMat &w, int64_t m);
hipError_t launch_gemm_kq_bf16(int id, const QMat &w, const uint16_t *x, float *y, int64_t m, float *ws, hipStream_t s);
hipError_t launch_synth_quant(int id, uint64_t seed, int64_t rows, int64_t cols, uint8_t *gguf,
                              hipStream_t s);
hipError_t launch_synth_f32(uint64_t seed, int64_t n, float *out, hipStream_t s);
hipError_t launch_synth_bf16(uint64_t seed, int64_t n, uint16_t *out, hipStream_t s);
hipError_t launch_spin(uint32_t microseconds, int wall_clock_khz, hipStream_t s);
hipError_t launch_copy(void *dst, const void *src, uint64_t nbytes, hipStream_t s);
// grid workgroups of 512 threads, `depth` (4 or 8) 1 KB loads in flight per wave; sink holds
// `grid` words (written only in a case no input produces in practice)
hipError_t launch_stream_read(const void *src, uint64_t nbytes, uint32_t *sink, int grid, int depth, hipStream_t s);
}  // namespace j4q

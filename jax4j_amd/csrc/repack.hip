// One-time layout kernels: GGUF blob -> split layout (repack), split -> GGUF (export),
// split -> fp32 rows (gather / full dequantization), and the seeded synthetic generators.
// None of these is on the timed path; they are byte-exact bijections or exact decodes.
#include "j4q_common.h"
#include "synth.h"

namespace j4q {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
__device__ __forceinline__ void st16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
__device__ __forceinline__ void st32(uint8_t *p, uint32_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
    p[2] = (uint8_t)(v >> 16);
    p[3] = (uint8_t)(v >> 24);
}
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Bit position, inside the Q6_K qh dword that serves ql dwords (2h, 2h+1) of a chunk, of
// the 2 high bits of the element held by byte b, nibble n of ql dword w (w = 0..3).
// Even dwords use bits {4..11, 20..27}; odd dwords the same pattern rotated by 8 bits.
// The GEMV recovers each fp16 pair with one AND plus one AND-OR (gemv.hip).
__host__ __device__ __forceinline__ int q6_hbit(int w, int b, int n) {
    const int pos = 4 + 2 * (b & 1) + 4 * n + 16 * (b >> 1);
    return (w & 1) ? ((pos + 8) & 31) : pos;
}

// ggml get_scale_min_k4 over the canonical 12 packed bytes.
__device__ __forceinline__ void k4_scale_min(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// One thread per GGUF block.
__global__ void __launch_bounds__(kThreads)
repack_kernel(int id, const uint8_t *__restrict__ src, uint8_t *__restrict__ base, int64_t rows, int64_t cols) {
    Geometry g;
    geometry_of(id, &g);
    const int64_t bpr = cols / g.block_elements;
    const int64_t bi = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (bi >= rows * bpr) return;
    const int64_t row = bi / bpr, j = bi % bpr;
    const uint8_t *b = src + bi * g.block_bytes;
    const QMat m = qmat_view(base, id, rows, cols);
    uint8_t *qs = const_cast<uint8_t *>(m.qs);
    uint8_t *sc = const_cast<uint8_t *>(m.sc);
    switch (id) {
    case Q4_0: {
        uint8_t *dst = qs + row * (cols / 2) + j * 16;
        for (int i = 0; i < 16; i++) dst[i] = b[2 + i];
        st16(sc + (row * bpr + j) * 2, ld16(b));
        break;
    }
    case Q8_0: {
        uint8_t *dst = qs + row * cols + j * 32;
        for (int i = 0; i < 32; i++) dst[i] = b[2 + i];
        st16(sc + (row * bpr + j) * 2, ld16(b));
        st16(const_cast<uint8_t *>(m.d) + (j * rows + row) * 2, ld16(b));
        break;
    }
    case Q2_0: {
        uint8_t *dst = qs + row * (cols / 4) + j * 32;
        for (int i = 0; i < 32; i++) dst[i] = b[2 + i];
        st16(sc + (row * bpr + j) * 2, ld16(b));
        break;
    }
    case Q4_K: {
        int s[8], mn[8];
        for (int t = 0; t < 8; t++) k4_scale_min(t, b + 4, s[t], mn[t]);
        uint32_t d0 = 0, d1 = 0, d2 = 0;
        for (int t = 0; t < 8; t++) {
            d0 |= (uint32_t)(s[t] & 15) << (4 * t);
            d1 |= (uint32_t)(mn[t] & 15) << (4 * t);
            d2 |= (uint32_t)(s[t] >> 4) << (2 * t);
            d2 |= (uint32_t)(mn[t] >> 4) << (16 + 2 * t);
        }
        uint8_t *meta = sc + (row * bpr + j) * 16;
        st16(meta, ld16(b));
        st16(meta + 2, ld16(b + 2));
        st32(meta + 4, d0);
        st32(meta + 8, d1);
        st32(meta + 12, d2);
        const uint8_t *q = b + 16;
        uint8_t *dst = qs + row * (cols / 2) + j * 128;
        for (int t = 0; t < 8; t++) {  // sub-block t = elements 32t..32t+31
            const uint8_t *grp = q + 32 * (t / 2);
            const int shift = (t & 1) ? 4 : 0;
            for (int i = 0; i < 16; i++) {
                const int lo = (grp[i] >> shift) & 15, hi = (grp[i + 16] >> shift) & 15;
                dst[16 * t + i] = (uint8_t)(lo | (hi << 4));
            }
        }
        break;
    }
    case Q6_K: {
        uint8_t q6[256];
        const uint8_t *ql = b, *qh = b + 128;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const uint8_t a = ql[64 * h + l], c = ql[64 * h + 32 + l], e = qh[32 * h + l];
                q6[128 * h + l] = (uint8_t)((a & 15) | ((e & 3) << 4));
                q6[128 * h + 32 + l] = (uint8_t)((c & 15) | (((e >> 2) & 3) << 4));
                q6[128 * h + 64 + l] = (uint8_t)((a >> 4) | (((e >> 4) & 3) << 4));
                q6[128 * h + 96 + l] = (uint8_t)((c >> 4) | (((e >> 6) & 3) << 4));
            }
        uint8_t *dql = qs + row * (cols / 2) + j * 128;
        uint8_t *dqh = const_cast<uint8_t *>(m.qh) + row * (cols / 4) + j * 64;
        for (int t = 0; t < 8; t++) {
            const uint8_t *e = q6 + 32 * t;
            for (int i = 0; i < 16; i++) dql[16 * t + i] = (uint8_t)((e[i] & 15) | ((e[i + 16] & 15) << 4));
            uint32_t h[2] = {0, 0};
            for (int w = 0; w < 4; w++)
                for (int bb = 0; bb < 4; bb++)
                    for (int n = 0; n < 2; n++)
                        h[w >> 1] |= (uint32_t)(e[4 * w + bb + 16 * n] >> 4) << q6_hbit(w, bb, n);
            st32(dqh + 8 * t, h[0]);
            st32(dqh + 8 * t + 4, h[1]);
        }
        uint8_t *dsc = sc + row * (cols / 16) + j * 16;
        for (int i = 0; i < 16; i++) dsc[i] = b[192 + i];
        st16(const_cast<uint8_t *>(m.d) + (row * bpr + j) * 2, ld16(b + 208));
        break;
    }
    default: break;
    }
}

// Exact inverse of repack_kernel.
__global__ void __launch_bounds__(kThreads)
export_kernel(int id, const uint8_t *__restrict__ base, uint8_t *__restrict__ dst, int64_t rows, int64_t cols) {
    Geometry g;
    geometry_of(id, &g);
    const int64_t bpr = cols / g.block_elements;
    const int64_t bi = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (bi >= rows * bpr) return;
    const int64_t row = bi / bpr, j = bi % bpr;
    uint8_t *b = dst + bi * g.block_bytes;
    const QMat m = qmat_view(base, id, rows, cols);
    switch (id) {
    case Q4_0: {
        const uint8_t *s = m.qs + row * (cols / 2) + j * 16;
        for (int i = 0; i < 16; i++) b[2 + i] = s[i];
        st16(b, ld16(m.sc + (row * bpr + j) * 2));
        break;
    }
    case Q8_0: {
        const uint8_t *s = m.qs + row * cols + j * 32;
        for (int i = 0; i < 32; i++) b[2 + i] = s[i];
        st16(b, ld16(m.sc + (row * bpr + j) * 2));
        break;
    }
    case Q2_0: {
        const uint8_t *s = m.qs + row * (cols / 4) + j * 32;
        for (int i = 0; i < 32; i++) b[2 + i] = s[i];
        st16(b, ld16(m.sc + (row * bpr + j) * 2));
        break;
    }
    case Q4_K: {
        const uint8_t *meta = m.sc + (row * bpr + j) * 16;
        st16(b, ld16(meta));
        st16(b + 2, ld16(meta + 2));
        const uint32_t d0 = ld32(meta + 4), d1 = ld32(meta + 8), d2 = ld32(meta + 12);
        int s[8], mn[8];
        for (int t = 0; t < 8; t++) {
            s[t] = (int)(((d0 >> (4 * t)) & 15) | (((d2 >> (2 * t)) & 3) << 4));
            mn[t] = (int)(((d1 >> (4 * t)) & 15) | (((d2 >> (16 + 2 * t)) & 3) << 4));
        }
        uint8_t *sp = b + 4;
        for (int t = 0; t < 4; t++) {
            sp[t] = (uint8_t)((s[t] & 63) | ((s[t + 4] >> 4) << 6));
            sp[t + 4] = (uint8_t)((mn[t] & 63) | ((mn[t + 4] >> 4) << 6));
            sp[t + 8] = (uint8_t)((s[t + 4] & 15) | ((mn[t + 4] & 15) << 4));
        }
        const uint8_t *src = m.qs + row * (cols / 2) + j * 128;
        uint8_t *q = b + 16;
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                // element 64c+l lives in sub-block 2c, element 64c+32+l in sub-block 2c+1
                const int i = l & 15, up = l >> 4;
                const int lo = (src[16 * (2 * c) + i] >> (4 * up)) & 15;
                const int hi = (src[16 * (2 * c + 1) + i] >> (4 * up)) & 15;
                q[32 * c + l] = (uint8_t)(lo | (hi << 4));
            }
        break;
    }
    case Q6_K: {
        uint8_t q6[256];
        const uint8_t *sql = m.qs + row * (cols / 2) + j * 128;
        const uint8_t *sqh = m.qh + row * (cols / 4) + j * 64;
        for (int t = 0; t < 8; t++) {
            const uint32_t h[2] = {ld32(sqh + 8 * t), ld32(sqh + 8 * t + 4)};
            for (int w = 0; w < 4; w++)
                for (int bb = 0; bb < 4; bb++)
                    for (int n = 0; n < 2; n++) {
                        const int i = 4 * w + bb;
                        const int lo4 = (sql[16 * t + i] >> (4 * n)) & 15;
                        const int hi2 = (h[w >> 1] >> q6_hbit(w, bb, n)) & 3;
                        q6[32 * t + i + 16 * n] = (uint8_t)(lo4 | (hi2 << 4));
                    }
        }
        uint8_t *ql = b, *qh = b + 128;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const uint8_t *e = q6 + 128 * h;
                ql[64 * h + l] = (uint8_t)((e[l] & 15) | ((e[l + 64] & 15) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((e[l + 32] & 15) | ((e[l + 96] & 15) << 4));
                qh[32 * h + l] = (uint8_t)((e[l] >> 4) | ((e[l + 32] >> 4) << 2) | ((e[l + 64] >> 4) << 4) |
                                           ((e[l + 96] >> 4) << 6));
            }
        const uint8_t *ssc = m.sc + row * (cols / 16) + j * 16;
        for (int i = 0; i < 16; i++) b[192 + i] = ssc[i];
        st16(b + 208, ld16(m.d + (row * bpr + j) * 2));
        break;
    }
    default: break;
    }
}

// One thread per (row, 32-element chunk): exact fp32 values of the GGUF formulas.
__global__ void __launch_bounds__(kThreads)
dequant_kernel(int id, QMat m, int64_t row0, int64_t nrows, float *__restrict__ out) {
    const int64_t chunks = m.cols / 32;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= nrows * chunks) return;
    const int64_t r = t / chunks, c = t % chunks, row = row0 + r;
    const int64_t cols = m.cols;
    float *o = out + r * cols + c * 32;
    switch (id) {
    case Q4_0: {
        const float d = half_bits_to_float(ld16(m.sc + (row * chunks + c) * 2));
        const uint8_t *q = m.qs + row * (cols / 2) + c * 16;
        for (int i = 0; i < 16; i++) {
            o[i] = __fmul_rn(d, (float)((q[i] & 15) - 8));
            o[i + 16] = __fmul_rn(d, (float)((q[i] >> 4) - 8));
        }
        break;
    }
    case Q8_0: {
        const float d = half_bits_to_float(ld16(m.sc + (row * chunks + c) * 2));
        const int8_t *q = (const int8_t *)(m.qs + row * cols + c * 32);
        for (int i = 0; i < 32; i++) o[i] = __fmul_rn(d, (float)q[i]);
        break;
    }
    case Q2_0: {
        const float d = half_bits_to_float(ld16(m.sc + (row * (cols / 128) + c / 4) * 2));
        const uint8_t *q = m.qs + row * (cols / 4) + c * 8;
        for (int i = 0; i < 32; i++) o[i] = __fmul_rn(d, (float)(((q[i >> 2] >> (2 * (i & 3))) & 3) - 1));
        break;
    }
    case Q4_K: {
        const uint8_t *meta = m.sc + (row * (cols / 256) + c / 8) * 16;
        const float d = half_bits_to_float(ld16(meta)), dmin = half_bits_to_float(ld16(meta + 2));
        const uint32_t d0 = ld32(meta + 4), d1 = ld32(meta + 8), d2 = ld32(meta + 12);
        const int j = (int)(c & 7);
        const int sc = (int)(((d0 >> (4 * j)) & 15) | (((d2 >> (2 * j)) & 3) << 4));
        const int mn = (int)(((d1 >> (4 * j)) & 15) | (((d2 >> (16 + 2 * j)) & 3) << 4));
        const float d1f = __fmul_rn(d, (float)sc), m1f = __fmul_rn(dmin, (float)mn);
        const uint8_t *q = m.qs + row * (cols / 2) + c * 16;
        for (int i = 0; i < 16; i++) {
            o[i] = __fsub_rn(__fmul_rn(d1f, (float)(q[i] & 15)), m1f);
            o[i + 16] = __fsub_rn(__fmul_rn(d1f, (float)(q[i] >> 4)), m1f);
        }
        break;
    }
    case Q6_K: {
        const float d = half_bits_to_float(ld16(m.d + (row * (cols / 256) + c / 8) * 2));
        const int8_t *s = (const int8_t *)(m.sc + row * (cols / 16) + c * 2);
        const float da = __fmul_rn(d, (float)s[0]), db = __fmul_rn(d, (float)s[1]);
        const uint8_t *ql = m.qs + row * (cols / 2) + c * 16;
        const uint8_t *qh = m.qh + row * (cols / 4) + c * 8;
        const uint32_t h[2] = {ld32(qh), ld32(qh + 4)};
        for (int w = 0; w < 4; w++)
            for (int bb = 0; bb < 4; bb++)
                for (int n = 0; n < 2; n++) {
                    const int i = 4 * w + bb;
                    const int q = (int)(((ql[i] >> (4 * n)) & 15) | (((h[w >> 1] >> q6_hbit(w, bb, n)) & 3) << 4)) - 32;
                    o[i + 16 * n] = __fmul_rn(n ? db : da, (float)q);
                }
        break;
    }
    default: break;
    }
}

__global__ void __launch_bounds__(kThreads)
synth_quant_kernel(int id, uint64_t seed, int64_t nblocks, int64_t cols, int block_bytes, uint8_t *__restrict__ out) {
    const int64_t bi = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (bi >= nblocks) return;
    uint8_t tmp[256];
    const int nb = j4q_synth::synth_block(id, seed, (uint64_t)bi, cols, tmp);
    uint8_t *o = out + bi * block_bytes;
    for (int i = 0; i < nb; i++) o[i] = tmp[i];
}

__global__ void __launch_bounds__(kThreads) synth_f32_kernel(uint64_t seed, int64_t n, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = j4q_synth::synth_x(seed, (uint64_t)i);
}

__global__ void __launch_bounds__(kThreads) synth_bf16_kernel(uint64_t seed, int64_t n, uint16_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = j4q_synth::f32_to_bf16(j4q_synth::synth_x(seed, (uint64_t)i));
}

// One thread per (row, block): d[block][row] = sc[row][block].
__global__ void __launch_bounds__(kThreads) q8_scales_t_kernel(QMat m) {
    const int64_t bpr = m.cols / 32, n = m.rows * bpr;
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int64_t row = i / bpr, j = i % bpr;
    st16(const_cast<uint8_t *>(m.d) + (j * m.rows + row) * 2, ld16(m.sc + i * 2));
}

inline unsigned grid_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_repack(int id, const uint8_t *gguf, uint8_t *split, int64_t rows, int64_t cols, hipStream_t s) {
    Geometry g;
    if (!geometry_of(id, &g)) return hipErrorInvalidValue;
    const int64_t n = rows * (cols / g.block_elements);
    if (n == 0) return hipSuccess;
    repack_kernel<<<grid_for(n), kThreads, 0, s>>>(id, gguf, split, rows, cols);
    return hipGetLastError();
}

hipError_t launch_q8_scales_t(const QMat &m, hipStream_t s) {
    const int64_t n = m.rows * (m.cols / 32);
    if (n == 0) return hipSuccess;
    q8_scales_t_kernel<<<grid_for(n), kThreads, 0, s>>>(m);
    return hipGetLastError();
}

hipError_t launch_export(int id, const uint8_t *split, uint8_t *gguf, int64_t rows, int64_t cols, hipStream_t s) {
    Geometry g;
    if (!geometry_of(id, &g)) return hipErrorInvalidValue;
    const int64_t n = rows * (cols / g.block_elements);
    if (n == 0) return hipSuccess;
    export_kernel<<<grid_for(n), kThreads, 0, s>>>(id, split, gguf, rows, cols);
    return hipGetLastError();
}

hipError_t launch_dequant_rows(int id, const QMat &m, int64_t row0, int64_t nrows, float *out, hipStream_t s) {
    const int64_t n = nrows * (m.cols / 32);
    if (n == 0) return hipSuccess;
    dequant_kernel<<<grid_for(n), kThreads, 0, s>>>(id, m, row0, nrows, out);
    return hipGetLastError();
}

hipError_t launch_synth_quant(int id, uint64_t seed, int64_t rows, int64_t cols, uint8_t *gguf, hipStream_t s) {
    Geometry g;
    if (!geometry_of(id, &g)) return hipErrorInvalidValue;
    const int64_t n = rows * (cols / g.block_elements);
    if (n == 0) return hipSuccess;
    synth_quant_kernel<<<grid_for(n), kThreads, 0, s>>>(id, seed, n, cols, g.block_bytes, gguf);
    return hipGetLastError();
}

hipError_t launch_synth_f32(uint64_t seed, int64_t n, float *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    synth_f32_kernel<<<grid_for(n), kThreads, 0, s>>>(seed, n, out);
    return hipGetLastError();
}

hipError_t launch_synth_bf16(uint64_t seed, int64_t n, uint16_t *out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    synth_bf16_kernel<<<grid_for(n), kThreads, 0, s>>>(seed, n, out);
    return hipGetLastError();
}

}  // namespace j4q

// ---- benchmark support -------------------------------------------------------------------
namespace j4q {
namespace {
// Holds the stream for `ticks` of the constant-rate wall clock (bounded: it always exits),
// so a host can queue many short launches behind it and time them back to back.
__global__ void spin_kernel(uint64_t ticks) {
    const uint64_t t0 = wall_clock64();
    for (uint32_t guard = 0; guard < (1u << 30); guard++) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(127);
    }
}
}  // namespace

typedef uint32_t cu32x4 __attribute__((ext_vector_type(4)));

// Grid-stride 128-bit copy: reads and writes each byte exactly once.
__global__ void __launch_bounds__(256) copy_kernel(const cu32x4 *__restrict__ src, cu32x4 *__restrict__ dst, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_copy(void *dst, const void *src, uint64_t nbytes, hipStream_t s) {
    const uint64_t n16 = nbytes / 16;
    if (n16 == 0) return hipSuccess;
    const uint64_t want = (n16 + 255) / 256;
    copy_kernel<<<(unsigned)(want < 4096 ? want : 4096), 256, 0, s>>>((const cu32x4 *)src, (cu32x4 *)dst, n16);
    return hipGetLastError();
}

// Read-only streaming probe: wave w of the grid reads its own contiguous segment of `seg`
// bytes (a multiple of U KB) with 128-bit non-temporal buffer loads, 1 KB per load
// instruction and U in flight, and writes nothing but a per-workgroup value no input
// produces in practice (so the loads cannot be dropped). Offsets past nbytes are out of the
// buffer resource's range: those loads return zeros without touching memory. It measures
// the practical HBM read ceiling of one launch of a given size: the same dispatch, ramp and
// tail a GEMV launch of that many bytes pays.
template <int U>
__global__ void __launch_bounds__(512) stream_read_kernel(const void *src, uint32_t nbytes, uint32_t seg,
                                                          uint32_t *__restrict__ sink) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(src), (short)0, (int)nbytes, 0x00020000);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w = blockIdx.x * 8u + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t base = w * seg + lane * 16u;
    uint32_t acc = 0;
    for (uint32_t off = 0; off < seg; off += 1024u * U) {
        cu32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++)
            v[u] = __builtin_bit_cast(cu32x4, __builtin_amdgcn_raw_buffer_load_b128(r, base + off + 1024u * u, 0, 2));
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

// nbytes < 2^31 (32-bit buffer offsets; the caller checks); loads in flight 4 or 8.
hipError_t launch_stream_read(const void *src, uint64_t nbytes, uint32_t *sink, int grid, int depth, hipStream_t s) {
    if (nbytes == 0) return hipSuccess;
    if (nbytes >= 0x80000000ull || grid <= 0 || (depth != 4 && depth != 8)) return hipErrorInvalidValue;
    const uint64_t waves = (uint64_t)grid * 8, step = 1024ull * (uint64_t)depth;
    const uint64_t seg = (nbytes + waves * step - 1) / (waves * step) * step;
    if (depth == 8)
        stream_read_kernel<8><<<(unsigned)grid, 512, 0, s>>>(src, (uint32_t)nbytes, (uint32_t)seg, sink);
    else
        stream_read_kernel<4><<<(unsigned)grid, 512, 0, s>>>(src, (uint32_t)nbytes, (uint32_t)seg, sink);
    return hipGetLastError();
}

hipError_t launch_spin(uint32_t microseconds, int wall_clock_khz, hipStream_t s) {
    const uint64_t ticks = (uint64_t)microseconds * (uint64_t)(wall_clock_khz > 0 ? wall_clock_khz : 100000) / 1000u;
    spin_kernel<<<1, 64, 0, s>>>(ticks);
    return hipGetLastError();
}
}  // namespace j4q

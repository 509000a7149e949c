// Decode GEMV y[b, n] = sum_k W[n, k] x[b, k] (+ add[b, n]) over split-layout weights.
//
// HBM-bound: every weight byte is read exactly once with a 128-bit load, and no MFMA is used.
// Mapping: a workgroup of 4 waves; each wave owns R consecutive rows; lane l of the wave
// handles the 32-element chunks c = l, l+64, ... of all R rows, so one wave-wide load moves
// 64 x 16 contiguous bytes of one row. x is staged once per workgroup in LDS (fp32, rotated
// so the 8 float4 reads of a chunk hit distinct banks) together with its 16-element sums.
//
// Unpack: a nibble AND-masked into the low bits of a 16-bit half is an fp16 subnormal whose
// value is q * 2^-24 (q * 2^-20 for the high nibble of a byte). v_fma_mix_f32 multiplies it
// exactly by the fp32 x and accumulates in fp32, so 8 Q4 weights cost 5 bit operations
// plus 8 FMAs and x never leaves fp32. Per-chunk partial sums are rescaled once per chunk:
//   Q4_0: d * (sum q x - 8 sum x)          Q8_0: d * (sum (q+128) x - 128 sum x)
//   Q4_K: d*sc * sum q x - dmin*m * sum x  Q6_K: d*sc_g * (sum q x - 32 sum x) per 16-group
// The rows' partial sums are reduced across the wave with DPP row operations and readlane.
#include "j4q_common.h"

namespace j4q {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr float kTwo24 = 16777216.0f;

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

template <class T>
__device__ __forceinline__ T ldg_stream(const T *p) {
    return __builtin_nontemporal_load(p);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes, valid in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror: every lane holds its 16-lane row sum
    float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// x values of one chunk: xs[j] = x[32c + 4j .. 32c + 4j + 3].
struct XChunk {
    f32x4 v[8];
};

// Q4-style chunk (16 B, byte i: lo nibble elem i, hi nibble elem i+16). slo gathers elements
// 0..15 in units of 2^-24, shi elements 16..31 in units of 2^-20.
__device__ __forceinline__ void q4_dot(u32x4 q, const XChunk &x, float &slo, float &shi) {
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t v = q[w], t = v >> 8;
        const half2_t p0 = as_h2(v & 0x000F000Fu), p1 = as_h2(v & 0x00F000F0u);
        const half2_t p2 = as_h2(t & 0x000F000Fu), p3 = as_h2(t & 0x00F000F0u);
        const f32x4 a = x.v[w], b = x.v[4 + w];
        slo = __builtin_fmaf((float)p0.x, a.x, slo);
        slo = __builtin_fmaf((float)p2.x, a.y, slo);
        slo = __builtin_fmaf((float)p0.y, a.z, slo);
        slo = __builtin_fmaf((float)p2.y, a.w, slo);
        shi = __builtin_fmaf((float)p1.x, b.x, shi);
        shi = __builtin_fmaf((float)p3.x, b.y, shi);
        shi = __builtin_fmaf((float)p1.y, b.z, shi);
        shi = __builtin_fmaf((float)p3.y, b.w, shi);
    }
}

// Q6_K chunk: q4_dot plus the two high bits merged from the qh dwords (layout in repack.hip:
// even ql dwords take fields at bits {4..11, 20..27} of their qh dword, odd ones the same
// fields rotated right by 8).
__device__ __forceinline__ void q6_dot(u32x4 q, u32x2 h, const XChunk &x, float &slo, float &shi) {
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t v = q[w], t = v >> 8;
        const uint32_t hw = (w & 1) ? __builtin_amdgcn_alignbit(h[w >> 1], h[w >> 1], 8) : h[w >> 1];
        const uint32_t hs = hw >> 2;
        const half2_t p0 = as_h2((v & 0x000F000Fu) | (hw & 0x00300030u));
        const half2_t p1 = as_h2((v & 0x00F000F0u) | (hw & 0x03000300u));
        const half2_t p2 = as_h2((t & 0x000F000Fu) | (hs & 0x00300030u));
        const half2_t p3 = as_h2((t & 0x00F000F0u) | (hs & 0x03000300u));
        const f32x4 a = x.v[w], b = x.v[4 + w];
        slo = __builtin_fmaf((float)p0.x, a.x, slo);
        slo = __builtin_fmaf((float)p2.x, a.y, slo);
        slo = __builtin_fmaf((float)p0.y, a.z, slo);
        slo = __builtin_fmaf((float)p2.y, a.w, slo);
        shi = __builtin_fmaf((float)p1.x, b.x, shi);
        shi = __builtin_fmaf((float)p3.x, b.y, shi);
        shi = __builtin_fmaf((float)p1.y, b.z, shi);
        shi = __builtin_fmaf((float)p3.y, b.w, shi);
    }
}

// Q8_0 chunk (32 B, natural order). Bytes are biased to q+128 so they are unsigned fp16
// subnormals; s0 + s1 is sum (q+128) x in units of 2^-24.
__device__ __forceinline__ void q8_dot(u32x4 qa, u32x4 qb, const XChunk &x, float &s0, float &s1) {
#pragma unroll
    for (int w = 0; w < 8; w++) {
        const uint32_t u = (w < 4 ? qa[w] : qb[w - 4]) ^ 0x80808080u;
        const half2_t p0 = as_h2(u & 0x00FF00FFu), p1 = as_h2((u >> 8) & 0x00FF00FFu);
        const f32x4 a = x.v[w];
        s0 = __builtin_fmaf((float)p0.x, a.x, s0);
        s1 = __builtin_fmaf((float)p1.x, a.y, s1);
        s0 = __builtin_fmaf((float)p0.y, a.z, s0);
        s1 = __builtin_fmaf((float)p1.y, a.w, s1);
    }
}

// Q2_0 chunk: 8 bytes, byte p holds elements 4p..4p+3 at 2 bits each (units of 2^-24 after
// shifting each field down to bit 0 of a half).
__device__ __forceinline__ void q2_dot(u32x2 q, const XChunk &x, float &s0, float &s1) {
#pragma unroll
    for (int w = 0; w < 2; w++) {
        const uint32_t v = q[w];
#pragma unroll
        for (int bpair = 0; bpair < 2; bpair++) {
            // bytes 2*bpair and 2*bpair+1 -> elements 16w + 8*bpair + 0..7
            const uint32_t b = (v >> (16 * bpair)) & 0xFFFFu;
            const uint32_t lohalf = (b & 0xFFu) | ((b & 0xFF00u) << 8);  // byte0 -> half lo, byte1 -> half hi
            const half2_t e0 = as_h2(lohalf & 0x00030003u);
            const half2_t e1 = as_h2((lohalf >> 2) & 0x00030003u);
            const half2_t e2 = as_h2((lohalf >> 4) & 0x00030003u);
            const half2_t e3 = as_h2((lohalf >> 6) & 0x00030003u);
            const int j = 4 * w + 2 * bpair;  // float4 index of the first byte's 4 elements
            const f32x4 a = x.v[j], c = x.v[j + 1];
            s0 = __builtin_fmaf((float)e0.x, a.x, s0);
            s1 = __builtin_fmaf((float)e1.x, a.y, s1);
            s0 = __builtin_fmaf((float)e2.x, a.z, s0);
            s1 = __builtin_fmaf((float)e3.x, a.w, s1);
            s0 = __builtin_fmaf((float)e0.y, c.x, s0);
            s1 = __builtin_fmaf((float)e1.y, c.y, s1);
            s0 = __builtin_fmaf((float)e2.y, c.z, s0);
            s1 = __builtin_fmaf((float)e3.y, c.w, s1);
        }
    }
}

// LDS image of x for one batch row: x rotated per chunk, then sums of each 16 elements.
__device__ __forceinline__ int xs_slot(int64_t c, int j) { return (int)(c * 8 + ((j + c) & 7)); }

__device__ __forceinline__ void stage_x(const float *__restrict__ x, int64_t K, f32x4 *xs, float *s16) {
    const int64_t groups = K / 4;
    for (int64_t g = threadIdx.x; g < groups; g += kThreads) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(x + 4 * g);
        const int64_t c = g >> 3;
        xs[xs_slot(c, (int)(g & 7))] = v;
        float p = (v.x + v.y) + (v.z + v.w);
        p += dpp<0xB1>(p);
        p += dpp<0x4E>(p);
        if ((g & 3) == 0) s16[g >> 2] = p;
    }
}

template <int FMT>
struct Chunk;

// Loads and the per-chunk scale math of each format. `row` is a row index that is valid
// (the caller clamps), `c` a chunk index < K/32.
template <>
struct Chunk<Q4_0> {
    u32x4 q;
    uint16_t d;
    __device__ __forceinline__ void load(const QMat &m, int64_t row, int64_t c) {
        q = ldg_stream(reinterpret_cast<const u32x4 *>(m.qs + row * (m.cols / 2) + c * 16));
        d = ldg_stream(reinterpret_cast<const uint16_t *>(m.sc) + row * (m.cols / 32) + c);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc) const {
        float slo = 0.f, shi = 0.f;
        q4_dot(q, x, slo, shi);
        const float df = half_bits_to_float(d);
        const float t = __builtin_fmaf(shi, 0.0625f, slo);
        acc = __builtin_fmaf(-8.0f * df, sx.x + sx.y, acc);
        return __builtin_fmaf(df * kTwo24, t, acc);
    }
};

template <>
struct Chunk<Q8_0> {
    u32x4 qa, qb;
    uint16_t d;
    __device__ __forceinline__ void load(const QMat &m, int64_t row, int64_t c) {
        const u32x4 *p = reinterpret_cast<const u32x4 *>(m.qs + row * m.cols + c * 32);
        qa = ldg_stream(p);
        qb = ldg_stream(p + 1);
        d = ldg_stream(reinterpret_cast<const uint16_t *>(m.sc) + row * (m.cols / 32) + c);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc) const {
        float s0 = 0.f, s1 = 0.f;
        q8_dot(qa, qb, x, s0, s1);
        const float df = half_bits_to_float(d);
        acc = __builtin_fmaf(-128.0f * df, sx.x + sx.y, acc);
        return __builtin_fmaf(df * kTwo24, s0 + s1, acc);
    }
};

template <>
struct Chunk<Q4_K> {
    u32x4 q, meta;
    __device__ __forceinline__ void load(const QMat &m, int64_t row, int64_t c) {
        q = ldg_stream(reinterpret_cast<const u32x4 *>(m.qs + row * (m.cols / 2) + c * 16));
        meta = ldg_stream(reinterpret_cast<const u32x4 *>(m.sc + (row * (m.cols / 256) + (c >> 3)) * 16));
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc, int j) const {
        float slo = 0.f, shi = 0.f;
        q4_dot(q, x, slo, shi);
        const float d = half_bits_to_float(meta.x & 0xFFFFu), dmin = half_bits_to_float(meta.x >> 16);
        const uint32_t sc = __builtin_amdgcn_ubfe(meta.y, 4 * j, 4) | (__builtin_amdgcn_ubfe(meta.w, 2 * j, 2) << 4);
        const uint32_t mn = __builtin_amdgcn_ubfe(meta.z, 4 * j, 4) | (__builtin_amdgcn_ubfe(meta.w, 16 + 2 * j, 2) << 4);
        const float t = __builtin_fmaf(shi, 0.0625f, slo);
        acc = __builtin_fmaf(-(dmin * (float)mn), sx.x + sx.y, acc);
        return __builtin_fmaf(d * (float)sc * kTwo24, t, acc);
    }
};

template <>
struct Chunk<Q6_K> {
    u32x4 q;
    u32x2 h;
    uint16_t s;  // two int8 group scales
    uint16_t d;
    __device__ __forceinline__ void load(const QMat &m, int64_t row, int64_t c) {
        q = ldg_stream(reinterpret_cast<const u32x4 *>(m.qs + row * (m.cols / 2) + c * 16));
        h = ldg_stream(reinterpret_cast<const u32x2 *>(m.qh + row * (m.cols / 4) + c * 8));
        s = ldg_stream(reinterpret_cast<const uint16_t *>(m.sc + row * (m.cols / 16)) + c);
        d = ldg_stream(reinterpret_cast<const uint16_t *>(m.d) + row * (m.cols / 256) + (c >> 3));
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc) const {
        float slo = 0.f, shi = 0.f;
        q6_dot(q, h, x, slo, shi);
        const float df = half_bits_to_float(d);
        const float da = df * (float)(int8_t)(s & 0xFF), db = df * (float)(int8_t)(s >> 8);
        acc = __builtin_fmaf(da, __builtin_fmaf(slo, kTwo24, -32.0f * sx.x), acc);
        return __builtin_fmaf(db, __builtin_fmaf(shi, 1048576.0f, -32.0f * sx.y), acc);
    }
};

template <>
struct Chunk<Q2_0> {
    u32x2 q;
    uint16_t d;
    __device__ __forceinline__ void load(const QMat &m, int64_t row, int64_t c) {
        q = ldg_stream(reinterpret_cast<const u32x2 *>(m.qs + row * (m.cols / 4) + c * 8));
        d = ldg_stream(reinterpret_cast<const uint16_t *>(m.sc) + row * (m.cols / 128) + (c >> 2));
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc) const {
        float s0 = 0.f, s1 = 0.f;
        q2_dot(q, x, s0, s1);
        const float df = half_bits_to_float(d);
        acc = __builtin_fmaf(-df, sx.x + sx.y, acc);
        return __builtin_fmaf(df * kTwo24, s0 + s1, acc);
    }
};

template <int FMT, int R>
__device__ __forceinline__ void accumulate(const Chunk<FMT> (&ch)[R], const XChunk &x, f32x2 sx, int j,
                                           float (&acc)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        if constexpr (FMT == Q4_K)
            acc[r] = ch[r].apply(x, sx, acc[r], j);
        else
            acc[r] = ch[r].apply(x, sx, acc[r]);
    }
}

// grid: (ceil(N / (kWaves*R)), batch). Dynamic LDS: K floats of x + K/16 sums.
template <int FMT, int R>
__global__ void __launch_bounds__(kThreads)
gemv_kernel(QMat m, const float *__restrict__ x, const float *__restrict__ add, float *__restrict__ y) {
    extern __shared__ f32x4 lds[];
    const int64_t K = m.cols, N = m.rows;
    const int64_t b = blockIdx.y;
    f32x4 *xs = lds;
    float *s16 = reinterpret_cast<float *>(lds + K / 4);
    stage_x(x + b * K, K, xs, s16);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row0 = ((int64_t)blockIdx.x * kWaves + wave) * R;
    int64_t rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) rows[r] = row0 + r < N ? row0 + r : N - 1;

    const int64_t nchunks = K / 32;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;

    Chunk<FMT> ch[R];
    int64_t c = lane;
    if (c < nchunks) {
#pragma unroll
        for (int r = 0; r < R; r++) ch[r].load(m, rows[r], c);
    }
    __syncthreads();
    const float2 *s16v = reinterpret_cast<const float2 *>(s16);
    while (c < nchunks) {
        // software pipeline: issue the next chunk's loads before consuming this one
        Chunk<FMT> nx[R];
        const int64_t cn = c + 64;
        if (cn < nchunks) {
#pragma unroll
            for (int r = 0; r < R; r++) nx[r].load(m, rows[r], cn);
        }
        XChunk xc;
#pragma unroll
        for (int j = 0; j < 8; j++) xc.v[j] = xs[xs_slot(c, j)];
        const float2 sv = s16v[c];
        accumulate<FMT, R>(ch, xc, f32x2{sv.x, sv.y}, (int)(c & 7), acc);
#pragma unroll
        for (int r = 0; r < R; r++) ch[r] = nx[r];
        c = cn;
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = wave_sum(acc[r]);
        if (lane == 0 && row0 + r < N) {
            const int64_t o = b * N + row0 + r;
            y[o] = add ? v + add[o] : v;
        }
    }
}

template <int FMT, int R>
hipError_t launch_fmt_r(const QMat &m, const float *x, const float *add, float *y, int64_t batch, hipStream_t s) {
    const int64_t rows_per_wg = (int64_t)kWaves * R;
    const dim3 grid((unsigned)((m.rows + rows_per_wg - 1) / rows_per_wg), (unsigned)batch);
    const size_t lds = (size_t)m.cols * 4 + (size_t)(m.cols / 16) * 4;
    gemv_kernel<FMT, R><<<grid, kThreads, lds, s>>>(m, x, add, y);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_fmt(const QMat &m, const float *x, const float *add, float *y, int64_t batch, hipStream_t s) {
    // Widest row group that still gives >= 2 workgroups per CU (256 CUs).
    const int64_t N = m.rows;
    if (N >= 4 * 4 * 512) return launch_fmt_r<FMT, 4>(m, x, add, y, batch, s);
    if (N >= 4 * 2 * 512) return launch_fmt_r<FMT, 2>(m, x, add, y, batch, s);
    return launch_fmt_r<FMT, 1>(m, x, add, y, batch, s);
}

}  // namespace

// Largest K whose x image fits the 64 KiB of LDS a workgroup may request.
int64_t gemv_max_cols() { return 15360; }

hipError_t launch_gemv(int id, const QMat &m, const float *x, const float *add, float *y, int64_t batch,
                       hipStream_t s) {
    if (m.rows <= 0 || batch <= 0) return hipSuccess;
    if (m.cols > gemv_max_cols() || batch > 65535) return hipErrorInvalidValue;
    switch (id) {
    case Q4_0: return launch_fmt<Q4_0>(m, x, add, y, batch, s);
    case Q8_0: return launch_fmt<Q8_0>(m, x, add, y, batch, s);
    case Q4_K: return launch_fmt<Q4_K>(m, x, add, y, batch, s);
    case Q6_K: return launch_fmt<Q6_K>(m, x, add, y, batch, s);
    case Q2_0: return launch_fmt<Q2_0>(m, x, add, y, batch, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace j4q

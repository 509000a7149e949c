// Decode GEMV y[n] = sum_k W[n, k] x[k] (+ add[n]) over split-layout weights (batch 1).
//
// HBM-bound: every weight byte is read exactly once with a buffer load (128-bit for the
// quant payload), and no MFMA is used. The kernel is persistent: a grid of a few hundred
// workgroups stages x once into LDS, then each wave streams row groups of R consecutive rows,
// either a fixed share g = wave, wave + total_waves, ... or (DYN) the next group of its
// workgroup's share from a pool in LDS. Lane l handles the 32-element chunks
// c = l, l + 64, ... of the group's rows, so one wave-wide load moves 64 x 16 contiguous bytes
// of a row. Work items (group, chunk step) form one flat stream per wave; the loads of item
// i + 1 are in flight while item i is computed, and the first item's loads are issued before
// x is staged, so the HBM stream starts at the top of the kernel.
//
// Unpack: a nibble AND-masked into the low bits of a 16-bit half is an fp16 subnormal whose
// value is q * 2^-24 (q * 2^-20 for the high nibble of a byte). v_fma_mix_f32 multiplies it
// exactly by the fp32 x and accumulates in fp32, so 8 Q4 weights cost 5 bit operations
// plus 8 FMAs and x never leaves fp32. Per-chunk partial sums are rescaled once per chunk:
//   Q4_0: d * (sum q x - 8 sum x)          Q8_0: d * (sum (q+128) x - 128 sum x)
//   Q4_K: d*sc * sum q x - dmin*m * sum x  Q6_K: d*sc_g * (sum q x - 32 sum x) per 16-group
// The rows' partial sums are reduced across the wave with DPP row operations and readlane.
//
// Addressing: each section of a matrix is a buffer resource (base in SGPRs; reads beyond
// the section return 0 without touching memory). A load's byte offset is a per-lane
// constant (VGPR, set once) plus a wave-uniform row/step offset (SGPR, scalar ALU), so the
// vector ALU spends nothing on addresses. x sits in LDS as [j][chunk] float4 slots with a
// compile-time stride NP, so the 8 reads of a chunk are one base plus immediate offsets,
// and consecutive lanes read consecutive 16-byte slots (no bank conflicts).
#pragma once

#include "j4q_common.h"

namespace j4q {
namespace gemv {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kTwo24 = 16777216.0f;
// Byte offset that is out of range for every buffer resource: loads from it return 0.
constexpr uint32_t kOob = 0x80000000u;
// Buffer load cache policy: non-temporal (weights are streamed once).
constexpr int kStream = 2;

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

// Device view of one matrix as buffer resources.
struct Rsrc {
    __amdgpu_buffer_rsrc_t qs, qh, sc, d;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffull ? 0x7fffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}

// `vo` is the per-lane byte offset, `so` the wave-uniform one.
__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, kStream));
}
__device__ __forceinline__ u32x2 ld64(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, kStream));
}
__device__ __forceinline__ uint32_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, kStream);
}

// Per-section byte offsets: per lane (within one 64-chunk step), per row and per step.
struct Offs {
    uint32_t qs, qh, sc, d;
};

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
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// x values of one chunk: v[j] = x[32c + 4j .. 32c + 4j + 3].
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

// LDS image of x for chunk stride NP (>= K/32): float4 slot j * NP + c holds
// x[32c + 4j .. 32c + 4j + 3]; after the 8 * NP slots, a float2 per chunk holds the sums of
// its two 16-element halves.
template <int NP>
struct XImage {
    static constexpr int kBytes = 8 * NP * 16 + NP * 8;
};

// x staging in two halves. load() issues all of a thread's x loads (XU float4, out-of-range
// slots read zeros); store() writes them to LDS with the 16-element sums. The kernel issues
// its first weight loads between the two: the vector-memory counter retires in order, so
// waiting for x (issued first) leaves those weight loads in flight.
template <int THREADS, int XU, int NP>
struct XStage {
    f32x4 v[XU];
    __device__ __forceinline__ void load(const float *__restrict__ x, int K) {
        const int groups = K / 4;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint64_t)K * 4);
#pragma unroll
        for (int u = 0; u < XU; u++) {
            const int g = (int)threadIdx.x + u * THREADS;
            v[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, g < groups ? 16u * g : kOob, 0, 0));
        }
    }
    __device__ __forceinline__ void store(int K, f32x4 *xs, float *s16) const {
        const int groups = K / 4;
#pragma unroll
        for (int u = 0; u < XU; u++) {
            const int g = (int)threadIdx.x + u * THREADS;
            float p = (v[u].x + v[u].y) + (v[u].z + v[u].w);
            p += dpp<0xB1>(p);
            p += dpp<0x4E>(p);
            if (g < groups) {
                xs[(g & 7) * NP + (g >> 3)] = v[u];
                if ((g & 3) == 0) s16[g >> 2] = p;
            }
        }
    }
};

// Section offsets of each format: per lane (chunk = lane within a 64-chunk step), per row
// and per 64-chunk step, for a matrix with K columns.
template <int FMT>
__device__ __forceinline__ void offsets(int K, int lane, Offs &ln, Offs &row, Offs &step) {
    const uint32_t k = (uint32_t)K, l = (uint32_t)lane;
    ln = Offs{0, 0, 0, 0};
    row = Offs{0, 0, 0, 0};
    step = Offs{0, 0, 0, 0};
    switch (FMT) {
    case Q4_0: ln = {16 * l, 0, 2 * l, 0}; row = {k / 2, 0, k / 16, 0}; step = {1024, 0, 128, 0}; break;
    case Q8_0: ln = {32 * l, 0, 2 * l, 0}; row = {k, 0, k / 16, 0}; step = {2048, 0, 128, 0}; break;
    case Q4_K: ln = {16 * l, 0, (l >> 3) * 16, 0}; row = {k / 2, 0, k / 16, 0}; step = {1024, 0, 128, 0}; break;
    case Q6_K:
        ln = {16 * l, 8 * l, 2 * l, (l >> 3) * 2};
        row = {k / 2, k / 4, k / 16, k / 128};
        step = {1024, 512, 128, 16};
        break;
    case Q2_0: ln = {8 * l, 0, (l >> 2) * 2, 0}; row = {k / 4, 0, k / 64, 0}; step = {512, 0, 32, 0}; break;
    default: break;
    }
}

template <int FMT>
struct Chunk;

// Loads and the per-chunk scale math of each format. `so` holds the wave-uniform offsets
// of the chunk's row and step; `j` (Q4_K) is the chunk's sub-block within its superblock.
// A loaded register read through an empty volatile asm where it is first used: the
// compiler otherwise hoisted the unpacking of a set's scales into the previous iteration,
// right behind the loads that fill them, and waited there for those loads (Q6_K: an HBM
// round trip every other item).
template <class T>
__device__ __forceinline__ T at_use(T v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <>
struct Chunk<Q4_0> {
    u32x4 q;
    uint32_t d;
    __device__ __forceinline__ void load(const Rsrc &r, const Offs &ln, const Offs &so) {
        q = ld128(r.qs, ln.qs, so.qs);
        d = ld16(r.sc, ln.sc, so.sc);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc, int) const {
        float slo = 0.f, shi = 0.f;
        q4_dot(q, x, slo, shi);
        const float df = half_bits_to_float(at_use(d));
        const float t = __builtin_fmaf(shi, 0.0625f, slo);
        acc = __builtin_fmaf(-8.0f * df, sx.x + sx.y, acc);
        return __builtin_fmaf(df * kTwo24, t, acc);
    }
};

template <>
struct Chunk<Q8_0> {
    u32x4 qa, qb;
    uint32_t d;
    __device__ __forceinline__ void load(const Rsrc &r, const Offs &ln, const Offs &so) {
        qa = ld128(r.qs, ln.qs, so.qs);
        qb = ld128(r.qs, ln.qs + 16u, so.qs);
        d = ld16(r.sc, ln.sc, so.sc);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc, int) const {
        float s0 = 0.f, s1 = 0.f;
        q8_dot(qa, qb, x, s0, s1);
        const float df = half_bits_to_float(at_use(d));
        acc = __builtin_fmaf(-128.0f * df, sx.x + sx.y, acc);
        return __builtin_fmaf(df * kTwo24, s0 + s1, acc);
    }
};

template <>
struct Chunk<Q4_K> {
    u32x4 q, meta;
    __device__ __forceinline__ void load(const Rsrc &r, const Offs &ln, const Offs &so) {
        q = ld128(r.qs, ln.qs, so.qs);
        meta = ld128(r.sc, ln.sc, so.sc);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc, int j) const {
        float slo = 0.f, shi = 0.f;
        q4_dot(q, x, slo, shi);
        const u32x4 meta = at_use(this->meta);
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
    uint32_t s;  // two int8 group scales
    uint32_t d;
    __device__ __forceinline__ void load(const Rsrc &r, const Offs &ln, const Offs &so) {
        q = ld128(r.qs, ln.qs, so.qs);
        h = ld64(r.qh, ln.qh, so.qh);
        s = ld16(r.sc, ln.sc, so.sc);
        d = ld16(r.d, ln.d, so.d);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc, int) const {
        float slo = 0.f, shi = 0.f;
        q6_dot(q, h, x, slo, shi);
        const uint32_t s = at_use(this->s);
        const float df = half_bits_to_float(at_use(d));
        const float da = df * (float)(int8_t)(s & 0xFF), db = df * (float)(int8_t)(s >> 8);
        // sum (q - 32) x stays in the fields' units (2^-24 low, 2^-20 high) and the restoring
        // power of two rides on the scale: sum (q - 32) x itself exceeds fp32 for |x| above
        // ~6e35 where d * sc * sum (q - 32) x does not. Powers of two scale exactly, so the
        // result is the same as restoring first.
        acc = __builtin_fmaf(da * kTwo24, __builtin_fmaf(sx.x, -0x1p-19f, slo), acc);
        return __builtin_fmaf(db * 1048576.0f, __builtin_fmaf(sx.y, -0x1p-15f, shi), acc);
    }
};

template <>
struct Chunk<Q2_0> {
    u32x2 q;
    uint32_t d;
    __device__ __forceinline__ void load(const Rsrc &r, const Offs &ln, const Offs &so) {
        q = ld64(r.qs, ln.qs, so.qs);
        d = ld16(r.sc, ln.sc, so.sc);
    }
    __device__ __forceinline__ float apply(const XChunk &x, f32x2 sx, float acc, int) const {
        float s0 = 0.f, s1 = 0.f;
        q2_dot(q, x, s0, s1);
        const float df = half_bits_to_float(at_use(d));
        acc = __builtin_fmaf(-df, sx.x + sx.y, acc);
        return __builtin_fmaf(df * kTwo24, s0 + s1, acc);
    }
};

// Buffer resources over the sections of a [rows, cols] split-layout matrix.
__device__ __forceinline__ Rsrc rsrc_of(const QMat &m, int fmt) {
    const SplitLayout L = split_layout(fmt, m.rows, m.cols);
    Rsrc r;
    r.qs = make_rsrc(m.qs, L.qs_bytes);
    r.qh = make_rsrc(m.qh ? m.qh : m.qs, m.qh ? L.qh_bytes : 0);
    r.sc = make_rsrc(m.sc, L.sc_bytes);
    r.d = make_rsrc(m.d ? m.d : m.qs, m.d ? L.d_bytes : 0);
    return r;
}

// grid: (G workgroups of WAVES waves, batch); groups = ceil(N / R). Dynamic LDS:
// XImage<NP>::kBytes. The launch covers the column window [2048 st0, 2048 st0 + KW) of every
// row: y = (W[:, window] x[window] + prev) + add, so a K wider than one x image runs as
// windows chained through prev (the previous window's y, read by the wave that rewrites that
// element) with the caller's add joining only in the last window. Requires KW % 32 == 0,
// KW / 32 <= NP, KW / 4 <= XU * WAVES * 64 and every section < 2^31 bytes.
// Optional per-wave timeline of a launch (engine-local measurement, j4q_gemv_trace): with
// `p` set, wave w < waves of the first batch row writes p[4 w ..] = {wall clock at entry,
// after x is staged, after its last item, items | (hardware CU id << 32)}; null: no trace.
struct TraceSink {
    uint64_t *p;
    int waves;
};
extern TraceSink g_gemv_trace;

// DYN: the workgroup's row groups form one pool that its waves take from through an LDS
// counter, one group at a time, instead of a fixed share per wave. The waves of a SIMD do
// not progress at one rate (the oldest is served first: with 14 items each, the four waves
// of a SIMD ended 9.4, 10.2, 11.7 and 12.7 us into a launch), so fixed shares end with the
// slowest wave; from the pool, the faster waves take more groups. Every group is still
// computed by one wave, its chunk steps in order, so results do not change. R = 1 only.
template <int FMT, int R, int WAVES, int D, int XU, int NP, bool DYN = false>
__global__ void __launch_bounds__(WAVES * 64)
gemv_kernel(QMat m, const float *__restrict__ x, const float *prev, const float *add, float *y, int groups, int st0,
            int KW, TraceSink trace) {
    static_assert(!DYN || (R == 1 && (NP == 128 || NP == 480)), "pooled groups: one row per group, x barrier");
    extern __shared__ f32x4 lds[];
    __shared__ int pool_next;  // DYN: the next pool index to hand out
    const uint64_t tt0 = trace.p ? wall_clock64() : 0;
    const int K = (int)m.cols, N = (int)m.rows;
    // blockIdx.y selects a batch row (each batch row streams W again; batched decode uses
    // the MFMA kernel instead).
    x += (int64_t)blockIdx.y * K + (int64_t)st0 * 2048;
    y += (int64_t)blockIdx.y * N;
    if (add) add += (int64_t)blockIdx.y * N;
    if (prev) prev += (int64_t)blockIdx.y * N;
    const int nchunks = KW / 32, cpl = (nchunks + 63) / 64;
    // The wave index is uniform; saying so keeps every row/step offset in SGPRs (a buffer
    // load with a VGPR soffset would need a waterfall loop).
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gw = (int)blockIdx.x * WAVES + wave, nw = (int)gridDim.x * WAVES;
    const int mine = gw < groups ? (groups - 1 - gw) / nw + 1 : 0;
    const int items = mine * cpl;
    const Rsrc rs = rsrc_of(m, FMT);
    Offs ln, rowb, stepb;
    offsets<FMT>(K, lane, ln, rowb, stepb);

    // Item i of this wave is (group gw + (i / cpl) * nw, chunk step i % cpl); lane l takes
    // chunk l + 64 * step of each of the group's R rows. Offsets beyond the rows' data are
    // harmless (they are never computed on); an item past the end reads from an
    // out-of-range offset, so it costs no memory traffic. Loads are unconditional: no branch
    // separates a load from its use, and each wait leaves the other sets' loads in flight.
    auto load_item = [&](int i, Chunk<FMT> (&ch)[R]) {
        const int q = i / cpl;
        const int st = i - q * cpl + st0;
        const int g = gw + q * nw;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = (uint32_t)(g * R + r < N ? g * R + r : N - 1);
            Offs so;
            so.qs = row * rowb.qs + (uint32_t)st * stepb.qs;
            so.qh = row * rowb.qh + (uint32_t)st * stepb.qh;
            so.sc = row * rowb.sc + (uint32_t)st * stepb.sc;
            so.d = row * rowb.d + (uint32_t)st * stepb.d;
            if (i >= items) so = Offs{kOob, kOob, kOob, kOob};
            ch[r].load(rs, ln, so);
        }
    };

    XStage<WAVES * 64, XU, NP> xst;
    xst.load(x, KW);
    // Windows of up to 4096 and of 8193..15360 columns: every wave of the workgroup issues its
    // x loads before any wave issues weight loads (the CU returns vector-memory data in issue
    // order, so x loads behind another wave's weight loads wait for those HBM misses). The
    // barrier waits for no memory. Measured in A/B pairs on one box: o (4096 x 4096 Q4_K) 5.41
    // -> 5.25 us, q|k|v 6.59 -> 6.42 us; down (K = 14336, one workgroup per CU) 11.62 -> 11.53
    // us once the set loads' waits were right (before that, 1-2 % slower with it).
    if constexpr (NP == 128 || NP == 480) {
        if constexpr (DYN) {
            // every wave starts with pool index = its wave index; the rest is handed out
            if (threadIdx.x == 0) pool_next = WAVES;
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the store is done before the barrier
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    // D register sets form a ring: set d holds items d, d + D, d + 2D, ...
    Chunk<FMT> set[D][R];
    // one set's loads after the other, as in the loop: with the sets' loads interleaved here
    // (q of both, then scales of both), the wait counts the compiler derives for the loop
    // from both paths into it waited, for a set's scales, for the next set's quants too
    // DYN: the load position (group lg or -1 when the wave's work is over, chunk step lst);
    // pool index k is group base + k % WAVES + (k / WAVES) nw, an increasing sequence, so the
    // groups below `groups` are a prefix of k and a wave stops at its first index past it.
    // A wave takes its next index when it starts loading a group (lane 0's LDS atomic) and
    // reads the result only when that group's loads are all issued, so the atomic's latency
    // hides behind a group's worth of items.
    const int base = (int)blockIdx.x * WAVES;
    int lg = gw < groups ? gw : -1, lst = 0, ktaken = 0;
    int sg[D], sst[D];  // ring slot d: group (-1: absent) and chunk step of its item
    auto load_next = [&](int d) __attribute__((always_inline)) {
        // a wave-uniform branch, then the lane test on its own: folded into one test, the
        // compiler computed (lst | lane) in the register of the row's pending y store and
        // waited for that store before every group
        if (lst == 0 && lg >= 0) {
            asm volatile("");
            if (lane == 0) ktaken = atomicAdd(&pool_next, 1);
        }
        sg[d] = lg;
        sst[d] = lst;
        const uint32_t row = (uint32_t)(lg >= 0 ? lg : 0);
        Offs so;
        so.qs = row * rowb.qs + (uint32_t)(lst + st0) * stepb.qs;
        so.qh = row * rowb.qh + (uint32_t)(lst + st0) * stepb.qh;
        so.sc = row * rowb.sc + (uint32_t)(lst + st0) * stepb.sc;
        so.d = row * rowb.d + (uint32_t)(lst + st0) * stepb.d;
        if (lg < 0) so = Offs{kOob, kOob, kOob, kOob};
        set[d][0].load(rs, ln, so);
        if (++lst == cpl) {
            lst = 0;
            if (lg >= 0) {
                const int k = __builtin_amdgcn_readfirstlane(ktaken);
                const int gn = base + k % WAVES + (k / WAVES) * nw;
                lg = gn < groups ? gn : -1;
            }
        }
    };
#pragma unroll
    for (int d = 0; d < D; d++) {
        if constexpr (DYN) load_next(d);
        else load_item(d, set[d]);
        __builtin_amdgcn_sched_barrier(0);
    }

    f32x4 *xs = lds;
    float *s16 = reinterpret_cast<float *>(lds + 8 * NP);
    xst.store(KW, xs, s16);
    __syncthreads();
    const uint64_t tt1 = trace.p ? wall_clock64() : 0;

    const float2 *s16v = reinterpret_cast<const float2 *>(s16);
    // Fixed shares: wave priority by the items the wave still has, so the waves a SIMD serves
    // last (its younger waves, with equal shares) catch up instead of ending the launch alone.
    // Measured (A/B pairs on one box): Q6_K 4096 x 14336 11.65-11.72 -> 11.15-11.27 us, decode
    // step B = 1 1.140-1.142 -> 1.130-1.131 ms. On the pooled kernel, where the pool already
    // balances the waves, it cost: o 4.68 -> 5.12 us, q|k|v 5.44 -> 5.82 us.
    auto set_prio = [](int left) __attribute__((always_inline)) {
        if (left > 5) __builtin_amdgcn_s_setprio(3);
        else if (left > 3) __builtin_amdgcn_s_setprio(2);
        else if (left > 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    };
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    int done = items;  // items this wave computed (trace)
    if constexpr (!DYN) {
        int step = 0, g = gw;
        auto process = [&](const Chunk<FMT>(&ch)[R]) {
            const int c = lane + 64 * step;
            if (c < nchunks) {
                XChunk xc;
                const f32x4 *xp = xs + c;
#pragma unroll
                for (int j = 0; j < 8; j++) xc.v[j] = xp[j * NP];
                const float2 sv = s16v[c];
#pragma unroll
                for (int r = 0; r < R; r++) acc[r] = ch[r].apply(xc, f32x2{sv.x, sv.y}, acc[r], lane & 7);
            }
            if (++step == cpl) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    float v = wave_sum(acc[r]);
                    const int row = __builtin_amdgcn_readfirstlane(g * R + r);
                    if (row < N) {
                        // wave-uniform addresses: scalar loads. prev may be y itself: this wave
                        // reads the element before its own lane 0 rewrites it.
                        if (prev) v += prev[row];
                        if (add) v += add[row];
                        if (lane == 0) y[row] = v;
                    }
                    acc[r] = 0.f;
                }
                step = 0;
                g += nw;
            }
        };
        // A set is only ever written by its own loads, so no in-flight load destination is
        // copied, and consuming set d waits only for its own loads: the D - 1 other sets stay in
        // flight.
        for (int i = 0; i < items; i += D) {
            set_prio(items - i);
#pragma unroll
            for (int d = 0; d < D; d++) {
                if (i + d < items) process(set[d]);
                load_item(i + d + D, set[d]);
            }
        }
    } else {
        auto process_slot = [&](int d) __attribute__((always_inline)) {
            const int c = lane + 64 * sst[d];
            if (c < nchunks) {
                XChunk xc;
                const f32x4 *xp = xs + c;
#pragma unroll
                for (int j = 0; j < 8; j++) xc.v[j] = xp[j * NP];
                const float2 sv = s16v[c];
                acc[0] = set[d][0].apply(xc, f32x2{sv.x, sv.y}, acc[0], lane & 7);
            }
            if (sst[d] == cpl - 1) {
                float v = wave_sum(acc[0]);
                const int row = sg[d];
                if (prev) v += prev[row];
                if (add) v += add[row];
                if (lane == 0) y[row] = v;
                acc[0] = 0.f;
            }
        };
        // items in load order, item i in slot i % D, in the shape of the fixed-share loop; the
        // first absent item ends the wave's work (every later one is absent too), so a round
        // that starts with an absent slot 0 is past the end
        done = 0;
        while (sg[0] >= 0) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                if (sg[d] >= 0) {
                    process_slot(d);
                    done++;
                }
                load_next(d);
            }
        }
    }
    if (trace.p && blockIdx.y == 0 && gw < trace.waves && lane == 0) {
        uint64_t *t = trace.p + 4 * (int64_t)gw;
        t[0] = tt0;
        t[1] = tt1;
        t[2] = wall_clock64();
        t[3] = (uint64_t)(uint32_t)done | ((uint64_t)__smid() << 32);
    }
}

template <int FMT, int R, int WAVES, int D, int XU, int NP, bool DYN = false>
hipError_t launch_k(const QMat &m, const float *x, const float *prev, const float *add, float *y, int batch, int grid,
                    int groups, int st0, int kw, hipStream_t s) {
    gemv_kernel<FMT, R, WAVES, D, XU, NP, DYN><<<dim3(grid, batch), WAVES * 64, XImage<NP>::kBytes, s>>>(
        m, x, prev, add, y, groups, st0, kw, g_gemv_trace);
    return hipGetLastError();
}

// Widest column window one launch covers: an x image of 32768 columns takes 139,264 bytes of
// the 160 KiB of LDS a workgroup may use.
constexpr int64_t kMaxWindow = 32768;

// One launch over the column window [c0, c0 + kw) (c0 a multiple of 2048). The kernel is
// instantiated for four x-image sizes: kw <= 4096, 8192, 15360 and 32768.
template <int FMT, int R, int WAVES, int D, bool DYN = false>
hipError_t launch(const QMat &m, const float *x, const float *prev, const float *add, float *y, int batch, int wg_cap,
                  int64_t c0, int64_t kw, hipStream_t s) {
    const int groups = (int)((m.rows + R - 1) / R);
    int grid = (groups + WAVES - 1) / WAVES;
    if (grid > wg_cap) grid = wg_cap;
    constexpr int T = WAVES * 64;
    const int st0 = (int)(c0 / 2048), k = (int)kw;
    if (c0 % 2048 != 0 || kw % 32 != 0 || kw <= 0) return hipErrorInvalidValue;
    if (kw <= 4096)
        return launch_k<FMT, R, WAVES, D, (1024 + T - 1) / T, 128, DYN>(m, x, prev, add, y, batch, grid, groups, st0, k, s);
    if constexpr (DYN) return hipErrorInvalidValue;  // pooled groups: windows of up to 4096 columns
    if (kw <= 8192) return launch_k<FMT, R, WAVES, D, (2048 + T - 1) / T, 256>(m, x, prev, add, y, batch, grid, groups, st0, k, s);
    if (kw <= 15360) return launch_k<FMT, R, WAVES, D, (3840 + T - 1) / T, 480>(m, x, prev, add, y, batch, grid, groups, st0, k, s);
    if (kw <= kMaxWindow) return launch_k<FMT, R, WAVES, D, (8192 + T - 1) / T, 1024>(m, x, prev, add, y, batch, grid, groups, st0, k, s);
    return hipErrorInvalidValue;
}

}  // namespace gemv
}  // namespace j4q

// Prefill GEMM over Q8_0 weights: Y[M, N] = X[M, K] . W[N, K]^T, fp32 output.
//
// Two MFMA variants over the same tiling (a workgroup of 4 waves as 2 x 2, each wave a
// (BM/2) x (BN/2) tile of 32 x 32 MFMA tiles; operands staged through LDS KB Q8_0 blocks at
// a time, rows padded by 16 bytes so the 16-byte fragment reads of 8 consecutive rows hit
// distinct banks):
//
//  int8: X is quantized per row and 32-element block (quantize_act below). One
//        v_mfma_i32_32x32x32_i8 covers exactly one Q8_0 block of a 32 x 32 tile; its int32
//        result is folded in block order as acc = fma(float(I), sx * dw, acc), the
//        arithmetic of the emulated reference, so results are bit-identical to it.
//  bf16: W is dequantized into LDS as bf16(d * q) (round to nearest even; d * q is exact in
//        fp32) and X is used as given; v_mfma_f32_32x32x16_bf16 accumulates the whole K in
//        fp32 with no per-block epilogue.
//
// MFMA operand layout (both variants): lane l supplies row (or column) l % 32 and the 16 bytes
// of k at 16 * (l / 32) within the instruction's k range; A and B use the same lane -> k map,
// so the hardware's order of k inside one instruction does not matter. Result element v of
// lane l is row 8 * (v / 4) + 4 * (l / 32) + v % 4, column l % 32.
#include "j4q_common.h"

namespace j4q {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffull ? 0x7fffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}
__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

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

// Row index of result element v of `lane` inside a 32 x 32 MFMA tile.
__device__ __forceinline__ int mfma_row(int lane, int v) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// ---- int8 variant --------------------------------------------------------------------------
// grid (ceil(N / BN), ceil(M / BM)), 256 threads. Requires K % 32 == 0. The next stage's
// global loads are issued into registers before the current stage is computed.
template <int BM, int BN, int KB>
__global__ void __launch_bounds__(256)
gemm_i8_kernel(QMat w, const int8_t *__restrict__ xq, const float *__restrict__ xs, float *__restrict__ y, int M) {
    constexpr int ROWB = KB * 32 + 16;
    constexpr int TM = BM / 64, TN = BN / 64;  // 32 x 32 tiles per wave
    constexpr int PIECES = (BM + BN) * KB * 2;  // 16-byte pieces per stage
    constexpr int PT = (PIECES + 255) / 256;
    constexpr int SC = (BM + BN) * KB;  // scales per stage
    constexpr int ST = (SC + 255) / 256;
    __shared__ __attribute__((aligned(16))) int8_t As[BM * ROWB];
    __shared__ __attribute__((aligned(16))) int8_t Bs[BN * ROWB];
    __shared__ __attribute__((aligned(16))) float Sx[KB][BM];
    __shared__ float Dw[KB][BN];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32;
    const int n0 = (int)blockIdx.x * BN, m0 = (int)blockIdx.y * BM;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(xq, (uint64_t)M * K);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(w.qs, (uint64_t)N * K);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(xs, (uint64_t)M * nblk * 4);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(w.sc, (uint64_t)N * nblk * 2);

    u32x4 pv[PT];
    uint32_t sv[ST];
    auto load_stage = [&](int kb0) {
#pragma unroll
        for (int t = 0; t < PT; t++) {
            const int p = tid + 256 * t;
            const bool isb = p >= BM * KB * 2;
            const int pp = isb ? p - BM * KB * 2 : p;
            const int r = pp / (KB * 2), piece = pp % (KB * 2);
            const int kbyte = kb0 * 32 + piece * 16;
            const int grow = (isb ? n0 : m0) + r;
            const bool ok = p < PIECES && grow < (isb ? N : M) && kbyte < K;
            pv[t] = ld128(isb ? rb : ra, ok ? (uint32_t)grow * (uint32_t)K + (uint32_t)kbyte : kOob);
        }
#pragma unroll
        for (int t = 0; t < ST; t++) {
            const int p = tid + 256 * t;
            if (p < BM * KB) {
                const int gm = m0 + p / KB, blk = kb0 + p % KB;
                const bool ok = gm < M && blk < nblk;
                sv[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? ((uint32_t)gm * nblk + blk) * 4u : kOob, 0, 0);
            } else {
                const int pp = p - BM * KB, gn = n0 + pp / KB, blk = kb0 + pp % KB;
                const bool ok = p < SC && gn < N && blk < nblk;
                sv[t] = __builtin_amdgcn_raw_buffer_load_b16(rd, ok ? ((uint32_t)gn * nblk + blk) * 2u : kOob, 0, 0);
            }
        }
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int t = 0; t < PT; t++) {
            const int p = tid + 256 * t;
            if (p < PIECES) {
                const bool isb = p >= BM * KB * 2;
                const int pp = isb ? p - BM * KB * 2 : p;
                const int r = pp / (KB * 2), piece = pp % (KB * 2);
                *reinterpret_cast<u32x4 *>((isb ? Bs : As) + r * ROWB + piece * 16) = pv[t];
            }
        }
#pragma unroll
        for (int t = 0; t < ST; t++) {
            const int p = tid + 256 * t;
            if (p < BM * KB) Sx[p % KB][p / KB] = __builtin_bit_cast(float, sv[t]);
            else if (p < SC) Dw[(p - BM * KB) % KB][(p - BM * KB) / KB] = half_bits_to_float(sv[t]);
        }
    };

    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.f;

    load_stage(0);
    for (int kb0 = 0; kb0 < nblk; kb0 += KB) {
        store_stage();
        __syncthreads();
        if (kb0 + KB < nblk) load_stage(kb0 + KB);
        const int kbn = nblk - kb0 < KB ? nblk - kb0 : KB;
        for (int kb = 0; kb < kbn; kb++) {
            i32x4 fa[TM], fb[TN];
            float dw[TN];
#pragma unroll
            for (int a = 0; a < TM; a++) {
                const int r = wm * (BM / 2) + a * 32 + (lane & 31);
                fa[a] = *reinterpret_cast<const i32x4 *>(As + r * ROWB + kb * 32 + (lane >> 5) * 16);
            }
#pragma unroll
            for (int b = 0; b < TN; b++) {
                const int c = wn * (BN / 2) + b * 32 + (lane & 31);
                fb[b] = *reinterpret_cast<const i32x4 *>(Bs + c * ROWB + kb * 32 + (lane >> 5) * 16);
                dw[b] = Dw[kb][c];
            }
#pragma unroll
            for (int a = 0; a < TM; a++) {
                float sx[16];
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const f32x4 t = *reinterpret_cast<const f32x4 *>(&Sx[kb][wm * (BM / 2) + a * 32 + 8 * g + 4 * (lane >> 5)]);
                    sx[4 * g] = t.x;
                    sx[4 * g + 1] = t.y;
                    sx[4 * g + 2] = t.z;
                    sx[4 * g + 3] = t.w;
                }
#pragma unroll
                for (int b = 0; b < TN; b++) {
                    const i32x16 zero = {};
                    const i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[a], fb[b], zero, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        acc[a][b][v] = __builtin_fmaf((float)I[v], __fmul_rn(sx[v], dw[b]), acc[a][b][v]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++) {
            const int col = n0 + wn * (BN / 2) + b * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm * (BM / 2) + a * 32 + mfma_row(lane, v);
                if (row < M && col < N) y[(int64_t)row * N + col] = acc[a][b][v];
            }
        }
}

// ---- bf16 variant --------------------------------------------------------------------------
// grid (ceil(N / BN), ceil(M / BM)), 256 threads. Requires K % 32 == 0. The next stage's
// global loads are issued into registers before the current stage is computed.
template <int BM, int BN, int KB>
__global__ void __launch_bounds__(256)
gemm_bf16_kernel(QMat w, const uint16_t *__restrict__ x, float *__restrict__ y, int M) {
    constexpr int ROWB = KB * 64 + 16;  // bf16 row bytes + pad
    constexpr int TM = BM / 64, TN = BN / 64;
    constexpr int AP = BM * KB * 4, APT = (AP + 255) / 256;  // A: 16-byte pieces (8 bf16)
    constexpr int BP = BN * KB * 2, BPT = (BP + 255) / 256;  // B: 16-byte pieces (16 int8)
    __shared__ __attribute__((aligned(16))) uint8_t As[BM * ROWB];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[BN * ROWB];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32;
    const int n0 = (int)blockIdx.x * BN, m0 = (int)blockIdx.y * BM;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(x, (uint64_t)M * K * 2);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(w.qs, (uint64_t)N * K);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(w.sc, (uint64_t)N * nblk * 2);

    u32x4 av[APT], bv[BPT];
    uint32_t dv[BPT];
    auto load_stage = [&](int kb0) {
#pragma unroll
        for (int t = 0; t < APT; t++) {
            const int p = tid + 256 * t;
            const int r = p / (KB * 4), piece = p % (KB * 4);
            const int kel = kb0 * 32 + piece * 8, gm = m0 + r;
            const bool ok = p < AP && gm < M && kel < K;
            av[t] = ld128(ra, ok ? ((uint32_t)gm * (uint32_t)K + (uint32_t)kel) * 2u : kOob);
        }
#pragma unroll
        for (int t = 0; t < BPT; t++) {
            const int p = tid + 256 * t;
            const int r = p / (KB * 2), piece = p % (KB * 2);
            const int blk = kb0 + piece / 2, gn = n0 + r;
            const bool ok = p < BP && gn < N && blk < nblk;
            bv[t] = ld128(rb, ok ? (uint32_t)gn * (uint32_t)K + (uint32_t)(kb0 * 32 + piece * 16) : kOob);
            dv[t] = __builtin_amdgcn_raw_buffer_load_b16(rd, ok ? ((uint32_t)gn * nblk + blk) * 2u : kOob, 0, 0);
        }
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int t = 0; t < APT; t++) {
            const int p = tid + 256 * t;
            if (p < AP) *reinterpret_cast<u32x4 *>(As + (p / (KB * 4)) * ROWB + (p % (KB * 4)) * 16) = av[t];
        }
#pragma unroll
        for (int t = 0; t < BPT; t++) {
            const int p = tid + 256 * t;
            if (p >= BP) continue;
            const float d = half_bits_to_float(dv[t]);
            u32x4 o[2];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t u = bv[t][j];
                const float f0 = d * (float)(int8_t)(u & 0xFF), f1 = d * (float)(int8_t)((u >> 8) & 0xFF);
                const float f2 = d * (float)(int8_t)((u >> 16) & 0xFF), f3 = d * (float)(int8_t)(u >> 24);
                const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f1) << 16);
                const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f2) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f3) << 16);
                o[j >> 1][(j & 1) * 2] = lo;
                o[j >> 1][(j & 1) * 2 + 1] = hi;
            }
            uint8_t *dst = Bs + (p / (KB * 2)) * ROWB + (p % (KB * 2)) * 32;
            reinterpret_cast<u32x4 *>(dst)[0] = o[0];
            reinterpret_cast<u32x4 *>(dst)[1] = o[1];
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++) acc[a][b] = f32x16{};

    load_stage(0);
    for (int kb0 = 0; kb0 < nblk; kb0 += KB) {
        store_stage();
        __syncthreads();
        if (kb0 + KB < nblk) load_stage(kb0 + KB);
        const int ksteps = (nblk - kb0 < KB ? nblk - kb0 : KB) * 2;  // 16-element MFMA steps
        for (int ks = 0; ks < ksteps; ks++) {
            bf16x8 fa[TM], fb[TN];
#pragma unroll
            for (int a = 0; a < TM; a++) {
                const int r = wm * (BM / 2) + a * 32 + (lane & 31);
                fa[a] = *reinterpret_cast<const bf16x8 *>(As + r * ROWB + ks * 32 + (lane >> 5) * 16);
            }
#pragma unroll
            for (int b = 0; b < TN; b++) {
                const int c = wn * (BN / 2) + b * 32 + (lane & 31);
                fb[b] = *reinterpret_cast<const bf16x8 *>(Bs + c * ROWB + ks * 32 + (lane >> 5) * 16);
            }
#pragma unroll
            for (int a = 0; a < TM; a++)
#pragma unroll
                for (int b = 0; b < TN; b++) acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++) {
            const int col = n0 + wn * (BN / 2) + b * 32 + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = m0 + wm * (BM / 2) + a * 32 + mfma_row(lane, v);
                if (row < M && col < N) y[(int64_t)row * N + col] = acc[a][b][v];
            }
        }
}

}  // namespace

hipError_t launch_quantize_act(const uint16_t *x, int64_t m, int64_t k, int8_t *q, float *scales, hipStream_t s) {
    const int64_t n = m * (k / 32);
    if (n == 0) return hipSuccess;
    quantize_act_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, m, k, q, scales);
    return hipGetLastError();
}

template <int BM, int BN, int KB>
hipError_t launch_i8(const QMat &w, const int8_t *xq, const float *xs, float *y, int64_t m, hipStream_t s) {
    const dim3 grid((unsigned)((w.rows + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    gemm_i8_kernel<BM, BN, KB><<<grid, 256, 0, s>>>(w, xq, xs, y, (int)m);
    return hipGetLastError();
}

template <int BM, int BN, int KB>
hipError_t launch_bf16(const QMat &w, const uint16_t *x, float *y, int64_t m, hipStream_t s) {
    const dim3 grid((unsigned)((w.rows + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    gemm_bf16_kernel<BM, BN, KB><<<grid, 256, 0, s>>>(w, x, y, (int)m);
    return hipGetLastError();
}

// Tile shape by M: small M gets small tiles so more workgroups stream W.
hipError_t launch_gemm_q8_int8(const QMat &w, const int8_t *xq, const float *xs, float *y, int64_t m, hipStream_t s) {
    if (m <= 0 || w.rows <= 0) return hipSuccess;
    if (m > 65535 * 64 || w.cols % 32 != 0 || (uint64_t)m * w.cols > 0x7fffffffull) return hipErrorInvalidValue;
    if (m <= 64) return launch_i8<64, 64, 4>(w, xq, xs, y, m, s);
    if (m <= 512) return launch_i8<64, 128, 4>(w, xq, xs, y, m, s);
    return launch_i8<128, 128, 4>(w, xq, xs, y, m, s);
}

hipError_t launch_gemm_q8_bf16(const QMat &w, const uint16_t *x, float *y, int64_t m, hipStream_t s) {
    if (m <= 0 || w.rows <= 0) return hipSuccess;
    if (m > 65535 * 64 || w.cols % 32 != 0 || (uint64_t)m * w.cols * 2 > 0x7fffffffull) return hipErrorInvalidValue;
    if (m <= 64) return launch_bf16<64, 64, 2>(w, x, y, m, s);
    if (m <= 512) return launch_bf16<64, 128, 2>(w, x, y, m, s);
    return launch_bf16<128, 128, 2>(w, x, y, m, s);
}

}  // namespace j4q

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
#include "gemm_wide.h"

namespace j4q {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
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

// Four lanes per (row, 32-element block): s = amax/127, q = clamp(roundf(x * (1/s)), +-127)
// (ggml quantize_row_q8_0 with the scale kept in fp32). Lane j of a quad takes elements
// 8 j .. 8 j + 7, so a wave reads 1 KB and writes 512 bytes contiguously; the quad's maximum
// comes from two DPP exchanges (max is exact in any order). Division and the reciprocal are
// IEEE correctly rounded, so the result is bit-identical to a C reference.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__global__ void __launch_bounds__(256)
quantize_act_kernel(const uint16_t *__restrict__ x, int64_t n16, int8_t *__restrict__ q, float *__restrict__ s) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte chunk of x
    const bool live = t < n16;
    const u32x4 p = live ? reinterpret_cast<const u32x4 *>(x)[t] : u32x4{0u, 0u, 0u, 0u};
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[2 * j] = __builtin_bit_cast(float, p[j] << 16);
        v[2 * j + 1] = __builtin_bit_cast(float, p[j] & 0xffff0000u);
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, dpp_f<0xB1>(amax));  // quad_perm [1,0,3,2]
    amax = fmaxf(amax, dpp_f<0x4E>(amax));  // quad_perm [2,3,0,1]
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    u32x2 out = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float r = __builtin_roundf(v[i] * id);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        out[i >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)r << (8 * (i & 3));
    }
    if (live) {
        reinterpret_cast<u32x2 *>(q)[t] = out;
        if ((threadIdx.x & 3) == 0) s[t >> 2] = d;
    }
}

// Row index of result element v of `lane` inside a 32 x 32 MFMA tile.
__device__ __forceinline__ int mfma_row(int lane, int v) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

// ---- the GEMM kernel (both variants) ------------------------------------------------------
// A workgroup of 4 waves (2 x 2) computes a BM x BN tile of Y over all of K in stages of KB
// Q8_0 blocks. Global loads run R stages ahead in a ring of R register sets (each set only
// ever written by its own loads, so no in-flight register is copied); a stage is written to
// one of two LDS buffers (the bf16 variant dequantizes W on the way), then one barrier, then
// the next loads are issued and the stage is computed. With two LDS buffers a single barrier
// per stage suffices: a buffer is rewritten only after every wave has passed the barrier
// that follows its last use.
enum { kVarInt8 = 0, kVarBf16 = 1 };

template <int VAR, int BM, int BN, int KB, int R, int G>
__global__ void __launch_bounds__(256 * G)
gemm_kernel(QMat w, const void *__restrict__ xv, const float *__restrict__ xs, float *__restrict__ y, int M) {
    constexpr int T = 256 * G;                      // threads
    constexpr int EB = VAR == kVarInt8 ? 1 : 2;     // bytes per activation element
    constexpr int AROW = KB * 32 * EB;              // A bytes per row per stage
    constexpr int BROW = KB * 32 * EB;              // B bytes per row per stage in LDS (bf16: dequantized)
    constexpr int ALD = AROW + 16, BLD = BROW + 16; // padded LDS row strides
    constexpr int TM = BM / 64, TN = BN / 64;       // 32 x 32 tiles per wave
    constexpr int AP = BM * AROW / 16, APT = (AP + T - 1) / T;  // A 16-byte pieces per stage
    constexpr int BP = BN * KB * 2, BPT = (BP + T - 1) / T;     // B 16-byte int8 pieces per stage
    constexpr int XP = VAR == kVarInt8 ? BM * KB : 0, XPT = (XP + T - 1) / T;  // activation scales
    // W scales: the int8 variant stages them in LDS (one slot per thread, no branch); the bf16
    // variant needs one per B piece for the dequantization.
    constexpr int DP = VAR == kVarInt8 ? BN * KB : BP, DPT = (DP + T - 1) / T;
    constexpr int ABUF = BM * ALD, BBUF = BN * BLD;
    __shared__ __attribute__((aligned(16))) uint8_t As[2][ABUF];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BBUF];
    __shared__ __attribute__((aligned(16))) float Sx[2][KB][VAR == kVarInt8 ? BM : 4];
    __shared__ float Dw[2][KB][VAR == kVarInt8 ? BN : 4];

    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32;
    const int nst = (nblk + KB - 1) / KB;
    // XCD-aware tile order: workgroup b runs on XCD b % 8, so when the tile count divides by 8
    // each XCD takes a contiguous range of tiles, M-fastest: the tiles one XCD runs at a time
    // share their W rows (and X) in that XCD's L2.
    const int mt = (M + BM - 1) / BM, tiles = (int)gridDim.x;
    int t = (int)blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
    const int n0 = (t / mt) * BN, m0 = (t % mt) * BM;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // waves 4g .. 4g+3 form group g (2 x 2 over the tile); group g computes its share of every
    // stage's k range, and the groups' partial tiles are added at the end
    const int grp = wave >> 2, wm = (wave & 3) >> 1, wn = wave & 1;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(xv, (uint64_t)M * K * EB);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(w.qs, (uint64_t)N * K);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(w.sc, (uint64_t)N * nblk * 2);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(xs, VAR == kVarInt8 ? (uint64_t)M * nblk * 4 : 0);

    struct Set {
        u32x4 a[APT], b[BPT];
        uint32_t d[DPT], x[XPT > 0 ? XPT : 1];
    };
    Set set[R];

    // Per-thread byte offsets of stage 0 (a stage advances every section by a wave-uniform
    // amount, passed as the buffer instruction's scalar offset). Pieces outside the matrix
    // get an out-of-range offset; pieces past K in the last stage read real bytes that the
    // compute never uses (it stops at the last block).
    uint32_t aoff[APT], boff[BPT], doff[DPT], xoff[XPT > 0 ? XPT : 1];
#pragma unroll
    for (int t = 0; t < APT; t++) {
        const int p = tid + T * t;
        const int r = p / (AROW / 16), piece = p % (AROW / 16), gm = m0 + r;
        aoff[t] = (p < AP && gm < M) ? (uint32_t)gm * (uint32_t)K * EB + (uint32_t)piece * 16u : kOob;
    }
#pragma unroll
    for (int t = 0; t < BPT; t++) {
        const int p = tid + T * t;
        const int r = p / (KB * 2), piece = p % (KB * 2), gn = n0 + r;
        const bool ok = p < BP && gn < N;
        boff[t] = ok ? (uint32_t)gn * (uint32_t)K + (uint32_t)piece * 16u : kOob;
        if constexpr (VAR == kVarBf16) doff[t] = ok ? ((uint32_t)gn * nblk + (uint32_t)(piece / 2)) * 2u : kOob;
    }
    if constexpr (VAR == kVarInt8) {
#pragma unroll
        for (int t = 0; t < DPT; t++) {
            const int p = tid + T * t, gn = n0 + p / KB;
            doff[t] = (p < DP && gn < N) ? ((uint32_t)gn * nblk + (uint32_t)(p % KB)) * 2u : kOob;
        }
    }
    if constexpr (VAR == kVarInt8) {
#pragma unroll
        for (int t = 0; t < XPT; t++) {
            const int p = tid + T * t, gm = m0 + p / KB;
            xoff[t] = (p < XP && gm < M) ? ((uint32_t)gm * nblk + (uint32_t)(p % KB)) * 4u : kOob;
        }
    }

    // Stage st's loads; stages past the end read an out-of-range offset (zeros, no traffic).
    auto load = [&](int st, Set &S) {
        const bool live = st < nst;
        const uint32_t kb0 = (uint32_t)(st * KB);
        const uint32_t sa = live ? kb0 * 32u * EB : kOob, sb = live ? kb0 * 32u : kOob;
        const uint32_t sd = live ? kb0 * 2u : kOob, sx = live ? kb0 * 4u : kOob;
#pragma unroll
        for (int t = 0; t < APT; t++)
            S.a[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, aoff[t], sa, 0));
#pragma unroll
        for (int t = 0; t < BPT; t++)
            S.b[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, boff[t], sb, 0));
#pragma unroll
        for (int t = 0; t < DPT; t++) S.d[t] = __builtin_amdgcn_raw_buffer_load_b16(rd, doff[t], sd, 0);
        if constexpr (VAR == kVarInt8) {
#pragma unroll
            for (int t = 0; t < XPT; t++) S.x[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, xoff[t], sx, 0);
        }
    };

    // Writes a stage into LDS buffer `bi`.
    auto store = [&](const Set &S, int bi) {
#pragma unroll
        for (int t = 0; t < APT; t++) {
            const int p = tid + T * t;
            if (APT * T == AP || p < AP) *reinterpret_cast<u32x4 *>(&As[bi][(p / (AROW / 16)) * ALD + (p % (AROW / 16)) * 16]) = S.a[t];
        }
#pragma unroll
        for (int t = 0; t < BPT; t++) {
            const int p = tid + T * t;
            if (BPT * T != BP && p >= BP) continue;
            const int r = p / (KB * 2), piece = p % (KB * 2);
            if constexpr (VAR == kVarInt8) {
                *reinterpret_cast<u32x4 *>(&Bs[bi][r * BLD + piece * 16]) = S.b[t];
            } else {
                // bf16(d * q): d * q is exact in fp32, the conversion rounds to nearest even
                const float d = half_bits_to_float(S.d[t]);
                u32x4 o[2];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t u = S.b[t][j];
                    const float f0 = d * (float)(int8_t)(u & 0xFF), f1 = d * (float)(int8_t)((u >> 8) & 0xFF);
                    const float f2 = d * (float)(int8_t)((u >> 16) & 0xFF), f3 = d * (float)(int8_t)(u >> 24);
                    o[j >> 1][(j & 1) * 2] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f0) |
                                             ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f1) << 16);
                    o[j >> 1][(j & 1) * 2 + 1] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f2) |
                                                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f3) << 16);
                }
                uint8_t *dst = &Bs[bi][r * BLD + piece * 32];
                reinterpret_cast<u32x4 *>(dst)[0] = o[0];
                reinterpret_cast<u32x4 *>(dst)[1] = o[1];
            }
        }
        if constexpr (VAR == kVarInt8) {
#pragma unroll
            for (int t = 0; t < XPT; t++) {
                const int p = tid + T * t;
                if (XPT * T == XP || p < XP) Sx[bi][p % KB][p / KB] = __builtin_bit_cast(float, S.x[t]);
            }
#pragma unroll
            for (int t = 0; t < DPT; t++) {
                const int p = tid + T * t;
                if (DPT * T == DP || p < DP) Dw[bi][p % KB][p / KB] = half_bits_to_float(S.d[t]);
            }
        }
    };

    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.f;

    // One Q8_0 block (int8) or one 16-element step (bf16) of a stage held in LDS buffer bi.
    auto step = [&](int bi, int k) {
        if constexpr (VAR == kVarInt8) {
            i32x4 fa[TM], fb[TN];
            float dw[TN];
#pragma unroll
            for (int a = 0; a < TM; a++) {
                const int r = wm * (BM / 2) + a * 32 + (lane & 31);
                fa[a] = *reinterpret_cast<const i32x4 *>(&As[bi][r * ALD + k * 32 + (lane >> 5) * 16]);
            }
#pragma unroll
            for (int b = 0; b < TN; b++) {
                const int c = wn * (BN / 2) + b * 32 + (lane & 31);
                fb[b] = *reinterpret_cast<const i32x4 *>(&Bs[bi][c * BLD + k * 32 + (lane >> 5) * 16]);
                dw[b] = Dw[bi][k][c];
            }
#pragma unroll
            for (int a = 0; a < TM; a++) {
                float sx[16];
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const f32x4 t = *reinterpret_cast<const f32x4 *>(&Sx[bi][k][wm * (BM / 2) + a * 32 + 8 * g + 4 * (lane >> 5)]);
                    sx[4 * g] = t.x;
                    sx[4 * g + 1] = t.y;
                    sx[4 * g + 2] = t.z;
                    sx[4 * g + 3] = t.w;
                }
                i32x16 I[TN];
#pragma unroll
                for (int b = 0; b < TN; b++) I[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[a], fb[b], i32x16{}, 0, 0, 0);
#pragma unroll
                for (int b = 0; b < TN; b++)
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        acc[a][b][v] = __builtin_fmaf((float)I[b][v], __fmul_rn(sx[v], dw[b]), acc[a][b][v]);
            }
        } else {
            bf16x8 fa[TM], fb[TN];
#pragma unroll
            for (int a = 0; a < TM; a++) {
                const int r = wm * (BM / 2) + a * 32 + (lane & 31);
                fa[a] = *reinterpret_cast<const bf16x8 *>(&As[bi][r * ALD + k * 32 + (lane >> 5) * 16]);
            }
#pragma unroll
            for (int b = 0; b < TN; b++) {
                const int c = wn * (BN / 2) + b * 32 + (lane & 31);
                fb[b] = *reinterpret_cast<const bf16x8 *>(&Bs[bi][c * BLD + k * 32 + (lane >> 5) * 16]);
            }
#pragma unroll
            for (int a = 0; a < TM; a++)
#pragma unroll
                for (int b = 0; b < TN; b++) {
                    f32x16 c;
#pragma unroll
                    for (int v = 0; v < 16; v++) c[v] = acc[a][b][v];
                    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], c, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[a][b][v] = c[v];
                }
        }
    };
    constexpr int KS = VAR == kVarInt8 ? KB : 2 * KB;  // steps per stage; group g takes [g KS/G, (g+1) KS/G)

    // Issue the prologue sets in ring order (the scheduler may not interleave them): the wait
    // before each store then counts exactly the younger sets' loads.
#pragma unroll
    for (int r = 0; r < R; r++) {
        load(r, set[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
    store(set[0], 0);
    // Iteration st: the barrier publishes stage st (stored during iteration st - 1) and frees
    // the other buffer (its last reader, stage st - 1, is done); then the loads R stages ahead
    // are issued, and stage st + 1 is dequantized/stored into the free buffer in the same
    // basic block as stage st's MFMAs, so VALU, LDS and MFMA work interleave. No early exit
    // inside the ring: a stage past the end loads nothing (out-of-range offsets) and computes
    // no blocks; an exit would make the wait before each store conservative (vmcnt(0)).
    for (int base = 0; base < nst; base += R) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int st = base + r;
            const int bi = st & 1;
            __syncthreads();
            load(st + R, set[r]);
            __builtin_amdgcn_sched_barrier(0);
            if (nblk - st * KB >= KB) {
                store(set[(r + 1) % R], bi ^ 1);
#pragma unroll
                for (int k = grp * KS / G; k < (grp + 1) * KS / G; k++) step(bi, k);
            } else {
                store(set[(r + 1) % R], bi ^ 1);
                const int kn = (nblk - st * KB) * (KS / KB);  // steps of a partial (or empty) stage
                for (int k = grp * KS / G; k < (grp + 1) * KS / G && k < kn; k++) step(bi, k);
            }
        }
    }

    if constexpr (G == 2) {
        // group 1 hands its partial tile to group 0 through LDS (the stage buffers are free
        // once every wave has passed this barrier); group 0 adds it in a fixed order
        static_assert(4 * TM * TN * 16 * 64 * 4 <= (int)sizeof(As), "reduction scratch");
        float *red = reinterpret_cast<float *>(&As[0][0]);
        __syncthreads();
        const int wq = wave & 3;
        if (grp == 1) {
#pragma unroll
            for (int a = 0; a < TM; a++)
#pragma unroll
                for (int b = 0; b < TN; b++)
#pragma unroll
                    for (int v = 0; v < 16; v++) red[(((wq * TM + a) * TN + b) * 16 + v) * 64 + lane] = acc[a][b][v];
        }
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int a = 0; a < TM; a++)
#pragma unroll
            for (int b = 0; b < TN; b++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[a][b][v] += red[(((wq * TM + a) * TN + b) * 16 + v) * 64 + lane];
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
    const int64_t n16 = m * (k / 8);  // 16-byte chunks: four per 32-element block
    if (n16 == 0) return hipSuccess;
    if ((n16 + 255) / 256 > 0x7fffffff) return hipErrorInvalidValue;
    quantize_act_kernel<<<(unsigned)((n16 + 255) / 256), 256, 0, s>>>(x, n16, q, scales);
    return hipGetLastError();
}

template <int VAR, int BM, int BN, int KB, int R, int G = 1>
hipError_t launch_gemm(const QMat &w, const void *x, const float *xs, float *y, int64_t m, hipStream_t s) {
    const uint64_t tiles = (uint64_t)((w.rows + BN - 1) / BN) * (uint64_t)((m + BM - 1) / BM);
    if (tiles > 0x7fffffffu) return hipErrorInvalidValue;
    gemm_kernel<VAR, BM, BN, KB, R, G><<<(unsigned)tiles, 256 * G, 0, s>>>(w, x, xs, y, (int)m);
    return hipGetLastError();
}

// Tile shape by M: small M gets small tiles so more workgroups stream W.
hipError_t launch_gemm_q8_int8(const QMat &w, const int8_t *xq, const float *xs, float *y, int64_t m, hipStream_t s) {
    if (m <= 0 || w.rows <= 0) return hipSuccess;
    if (m > 65535 * 64 || w.cols % 32 != 0 || (uint64_t)m * w.cols > 0x7fffffffull) return hipErrorInvalidValue;
    if (w.rows % 8 == 0 && (uint64_t)w.rows * w.cols <= 0x7fffffffull) {
        // gemm_wide.h, measured on MI355X at N = K = 4096: 16 x 32 tiles of 2 waves up to
        // M = 256 (M = 32 16.8 us against 33.1 on the 4-wave kernel, M = 128 23.3 against 36.0,
        // M = 256 35.0 against 37.0), 64 x 128 tiles of 8 waves above (M = 512 40.2 us against
        // 52.0, M = 2048 151 against 181)
        if (m <= 256) {
            const int64_t tiles = ((m + 15) / 16) * ((w.rows + 31) / 32);
            if (tiles > 0x7fffffff) return hipErrorInvalidValue;
            // four K ranges up to 256 tiles, one per CU of an MI355X (M = 32: 14.4 us against
            // 19.7); the bound is a constant so that results do not depend on the device
            if (tiles <= 256) gw::gemm_i8_small<4, 4><<<(unsigned)tiles, 512, 0, s>>>(w, xq, xs, y, (int)m);
            else gw::gemm_i8_small<4, 1><<<(unsigned)tiles, 128, 0, s>>>(w, xq, xs, y, (int)m);
        } else {
            const int64_t tiles = ((m + 63) / 64) * ((w.rows + 127) / 128);
            if (tiles > 0x7fffffff) return hipErrorInvalidValue;
            gw::gemm_i8_lds<<<(unsigned)tiles, 512, 0, s>>>(w, xq, xs, y, (int)m);
        }
        return hipGetLastError();
    }
    if (m <= 64) return launch_gemm<kVarInt8, 64, 64, 8, 3>(w, xq, xs, y, m, s);
    if (m <= 512) return launch_gemm<kVarInt8, 64, 128, 4, 4>(w, xq, xs, y, m, s);
    return launch_gemm<kVarInt8, 128, 128, 4, 3>(w, xq, xs, y, m, s);
}

hipError_t launch_gemm_q8_bf16(const QMat &w, const uint16_t *x, float *y, int64_t m, hipStream_t s) {
    if (m <= 0 || w.rows <= 0) return hipSuccess;
    if (m > 65535 * 64 || w.cols % 32 != 0 || (uint64_t)m * w.cols * 2 > 0x7fffffffull) return hipErrorInvalidValue;
    if (m > 64 && w.rows % 2 == 0 && (uint64_t)w.rows * w.cols <= 0x7fffffffull) {
        // gemm_wide.h, tiles loaded straight into LDS: the largest tile whose grid still
        // fills the GPU (measured on MI355X, K = 4096: M = 512, N = 4096 in 29-30 us at
        // 128 x 64; M = 2048 in 90 us at 128 x 128; M = 128..256, N = 4096 in 18.5-19.9 us at
        // 64 x 64, against 20.8-36.4 us on the small-M and 4-wave kernels; with fewer than 128
        // workgroups those kernels are faster: M = 64, or N = 1024 at M = 128)
        const int64_t nt64 = (w.rows + 63) / 64, nt128 = (w.rows + 127) / 128;
        const int64_t g128x128 = ((m + 127) / 128) * nt128, g128 = ((m + 127) / 128) * nt64, g64 = ((m + 63) / 64) * nt64;
        if (g64 > 0x7fffffff) return hipErrorInvalidValue;
        if (g128x128 >= 256) {
            gw::gemm_bf16_lds<128, 2, true><<<(unsigned)g128x128, 512, 0, s>>>(w, x, y, (int)m);
            return hipGetLastError();
        }
        if (g128 >= 192) {
            // the next stage's loads spread between the MFMAs here too, since the waves' priority
            // follows their place in the stage (A/B on one box, three rounds: M = 512 31.6-32.1 ->
            // 30.2-30.9 us; without the priority the spread did not pay at this tile)
            gw::gemm_bf16_lds<128, 1, true><<<(unsigned)g128, 512, 0, s>>>(w, x, y, (int)m);
            return hipGetLastError();
        }
        if (g64 >= 128) {
            gw::gemm_bf16_lds<64, 1, false><<<(unsigned)g64, 512, 0, s>>>(w, x, y, (int)m);
            return hipGetLastError();
        }
    }
    if (m >= 512 && (uint64_t)w.rows * w.cols <= 0x7fffffffull) {
        // gemm_wide.h, register-staged (odd N, or too few tiles for the kernel above): 128 x 128
        // tiles when they fill the GPU, else 128 x 64
        const int64_t mt = (m + 127) / 128, t128 = mt * ((w.rows + 127) / 128), t64 = mt * ((w.rows + 63) / 64);
        if (t64 > 0x7fffffff) return hipErrorInvalidValue;
        if (t128 >= 256) gw::gemm_bf16_wide<128, 2, 4><<<(unsigned)t128, 512, 0, s>>>(w, x, y, (int)m);
        else gw::gemm_bf16_wide<128, 1, 4><<<(unsigned)t64, 512, 0, s>>>(w, x, y, (int)m);
        return hipGetLastError();
    }
    if (m <= 192 && (uint64_t)w.rows * w.cols <= 0x7fffffffull) {
        // gemm_wide.h, small M: 16 weight rows per workgroup, all of K (measured on MI355X,
        // N = K = 4096: M = 32 in 11.7 us, M = 128 in 23.0 us with 64-row tiles, M = 192 in
        // 31.6 us against 34.1 on the 4-wave kernel; 128-row tiles are no faster at M = 128)
        const int64_t nt = (w.rows + 15) / 16, bm = m <= 32 ? 32 : 64;
        const int64_t grid = ((m + bm - 1) / bm) * nt;
        if (grid > 0x7fffffff) return hipErrorInvalidValue;
        if (bm == 32) gw::gemm_bf16_narrow<32, 2, 2><<<(unsigned)grid, 512, 0, s>>>(w, x, y, (int)m);
        else gw::gemm_bf16_narrow<64, 1, 2><<<(unsigned)grid, 512, 0, s>>>(w, x, y, (int)m);
        return hipGetLastError();
    }
    if (m <= 64) return launch_gemm<kVarBf16, 64, 64, 4, 3, 2>(w, x, nullptr, y, m, s);
    if (m <= 512) return launch_gemm<kVarBf16, 128, 64, 4, 3, 2>(w, x, nullptr, y, m, s);
    return launch_gemm<kVarBf16, 128, 128, 2, 3, 1>(w, x, nullptr, y, m, s);
}

}  // namespace j4q

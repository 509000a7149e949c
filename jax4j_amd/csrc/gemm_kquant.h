// Prefill GEMM, bf16 variant, over Q4_0, Q4_K and Q6_K weights: Y[M, N] = X[M, K] .
// bf16(W)[N, K]^T with fp32 accumulation, W the exactly decoded weights of the GGUF blocks
// (semantics: quantMatvec per row of X, QuantizedOps.java:27 / CpuBackend.java:708-725).
//
// Structure (shared with gemm_bf16_lds in gemm_wide.h, which serves Q8_0):
//  - Tile BM x 64 NJ per workgroup of 8 waves; wave w owns columns [16 NJ (w % 4), +16 NJ)
//    and 32-blocks 2 b + w / 4 (b = 0, 1) of every 128-k stage, for all BM rows; the two
//    waves of a column group add their partial tiles through LDS at the end.
//  - Every stage goes straight from global memory into one of three LDS stage buffers
//    (buffer_load ... lds, no VGPRs): X as BM rows x 256 bytes (16-byte chunk c of row r at
//    c ^ (r % 16)), the 4-bit quants of the split layout as BN rows x 64 bytes (chunk c of
//    row r at c ^ ((r / 4) % 4): the 16 rows of one operand read fall on distinct banks),
//    Q6_K's high-bit dwords as BN rows x 32 bytes, and each wave's per-row scale words of
//    the stage into its own 256-byte slot.
//  - MFMA lane group g = lane / 16 supplies k = 8 g .. 8 g + 7 of its block for A (X) and B
//    (W) alike. In the split layout byte i of a 32-element chunk holds element i (low
//    nibble) and element i + 16 (high nibble), so lane group g reads bytes 8 (g % 2) .. + 7
//    and takes their nibble g / 2: elements 8 g + 0 .. 7, in order.
//  - Each W element is dequantized once per workgroup, in the registers of the lane that
//    feeds it to the MFMA, to the fp32 value of the ggml decoder and then to bf16 (round to
//    nearest even):
//      Q4_0  w = d (q - 8)                 = fma(d, q, -8 d)       (exact)
//      Q4_K  w = fl((d sc) q - dmin m)     = fma(d sc, q, -dmin m) (d sc q is exact in fp32)
//      Q6_K  w = fl((d sc) (q - 32))       = fma(d sc, q, -32 d sc)
//    each FMA rounds the exact value once, as the decoder's operations do, so the bf16 weight
//    equals bf16 of the decoder's fp32 weight bit for bit.
//  - Iteration i: wait for own stage-i loads, barrier, load stage i + 2 into the buffers of
//    stage i - 1, read the operands of stage i, dequantize, run the MFMAs. Stages past the
//    end load zeros (out-of-range offsets: zero quants and zero scales decode to 0).
// grid = (ceil(M / BM) * ceil(N / (64 NJ)), S) workgroups of 512 threads: S K splits of
// split_stages stages each (S = 1: the whole of K, written to y; S > 1: partial tiles to
// part[s][M][N], added by sum_splits_kernel). Requires K % 128 == 0 (K % 256 for the
// K-quants), M * K * 2 < 2^31 and N * K / 2 < 2^31.
#pragma once

#include "gemm_wide.h"

namespace j4q {
namespace gk {

using gw::bf16x2;
using gw::bf16x8;
using gw::dma16;
using gw::dma4;
using gw::f32x2;
using gw::f32x4;
using gw::kOob;
using gw::lds_barrier;
using gw::make_rsrc;
using gw::u32x2;
using gw::u32x4;
using gw::wait_vm_lgkm0;

// Quant-tile swizzle: slot of 16-byte chunk c of row r is c ^ qswz(r).
__device__ __forceinline__ int qswz(int row) { return (row >> 2) & 3; }

__device__ __forceinline__ uint32_t rotr(uint32_t v, int s) { return __builtin_rotateright32(v, (uint32_t)s); }

// The four bytes of v as floats (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ void bytes_to_f32(uint32_t v, float &a, float &b, float &c, float &d) {
    a = (float)(v & 0xFFu);
    b = (float)((v >> 8) & 0xFFu);
    c = (float)((v >> 16) & 0xFFu);
    d = (float)(v >> 24);
}

// bf16(fma(s, q_i, o)) of the eight byte-sized codes in (lo, hi), packed as an MFMA operand.
__device__ __forceinline__ bf16x8 deq8(uint32_t lo, uint32_t hi, float s, float o) {
    u32x4 r;
    float f[8];
    bytes_to_f32(lo, f[0], f[1], f[2], f[3]);
    bytes_to_f32(hi, f[4], f[5], f[6], f[7]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = __builtin_fmaf(s, f[2 * i], o), b = __builtin_fmaf(s, f[2 * i + 1], o);
        r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2));
    }
    return __builtin_bit_cast(bf16x8, r);
}

// Q6_K: the two high bits of the four codes held by ql dword w of a chunk, moved to bits 4..5
// of each byte. h is the qh dword serving ql dwords (2 (w / 2), 2 (w / 2) + 1); the bit of
// byte b, nibble n sits at 4 + 2 (b % 2) + 4 n + 16 (b / 2) for even w and 8 bits further
// (mod 32) for odd w (repack.hip, q6_hbit).
__device__ __forceinline__ uint32_t q6_high(uint32_t h, int rot) {
    const uint32_t t = rotr(h, rot);
    return (t & 0x00300030u) | ((t << 6) & 0x30003000u);
}

template <int FMT, int BM, int NJ>
struct KqTile {
    static constexpr int BN = 64 * NJ, TM = BM / 16, XD = BM / 32;
    static constexpr int RW = BN / 8;                 // rows whose scale words one wave loads
    static constexpr int QHL = FMT == Q6_K ? NJ : 0;  // high-bit loads per wave and stage
    static constexpr int P = XD + 1 + QHL + 1;        // vector-memory instructions per wave and stage
    static constexpr int kX = BM * 256;
    static constexpr int kQ = BN * 64 + (NJ == 1 ? 1024 : 0);  // + a sink for the idle waves' loads
    static constexpr int kH = FMT == Q6_K ? BN * 32 : 16;
    static constexpr int kS = 8 * 256;
    static constexpr int kBytes = 3 * (kX + kQ + kH + kS);
    static_assert(kBytes <= 163840, "LDS");
};

template <int FMT, int BM, int NJ>
__global__ void __launch_bounds__(512)
gemm_kq_bf16(QMat w, const uint16_t *__restrict__ x, float *__restrict__ y, int M, int split_stages,
             float *__restrict__ part) {
    using T = KqTile<FMT, BM, NJ>;
    constexpr int BN = T::BN, TM = T::TM, XD = T::XD, RW = T::RW, QHL = T::QHL, P = T::P;
    __shared__ __attribute__((aligned(1024))) uint8_t xs0[T::kX], xs1[T::kX], xs2[T::kX];
    __shared__ __attribute__((aligned(1024))) uint8_t qs0[T::kQ], qs1[T::kQ], qs2[T::kQ];
    __shared__ __attribute__((aligned(256))) uint8_t hs0[T::kH], hs1[T::kH], hs2[T::kH];
    __shared__ __attribute__((aligned(256))) uint8_t ss0[T::kS], ss1[T::kS], ss2[T::kS];
    const int N = (int)w.rows, K = (int)w.cols;
    // K split: workgroup (tile, s) takes stages [s L, min((s + 1) L, K / 128)) (L =
    // split_stages) and writes its partial tile to part[s] when part is set (the splits are
    // added in order by sum_splits_kernel), else the tile itself to y
    const int sbeg = (int)blockIdx.y * split_stages, send0 = sbeg + split_stages;
    const int ns = send0 < K / 128 ? send0 : K / 128;  // stages at or past ns load nothing
    const int mt = (M + BM - 1) / BM;
    // Workgroup b runs on XCD b % 8; tile order is m fastest and each XCD takes a contiguous
    // range of it, so the m tiles of a group of n tiles (the same W rows) share an L2.
    const int total = (int)gridDim.x;
    int tile = (int)blockIdx.x;
    if (total % 8 == 0) tile = (tile % 8) * (total / 8) + tile / 8;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = wave & 3, kh = wave >> 2;  // column group, block parity
    const int m16 = lane & 15, g = lane >> 4;

    // X load j of this wave covers rows 4 (8 j + wave) .. +3; lane L fills LDS slot L % 16 of
    // row 4 (8 j + wave) + L / 16, which holds chunk (L % 16) ^ (row % 16).
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint64_t)M * (uint64_t)K * 2u);
    uint32_t xoff[XD];
    int xk[XD];
#pragma unroll
    for (int j = 0; j < XD; j++) {
        const int row = 4 * (8 * j + wave) + (lane >> 4), c = (lane & 15) ^ (row & 15), gm = m0 + row;
        xoff[j] = gm < M ? (uint32_t)gm * (uint32_t)K * 2u + (uint32_t)c * 16u : kOob;
        xk[j] = c * 8;
    }
    // Quants: wave w < BN / 16 loads rows 16 w .. 16 w + 15, lane L slot L % 4 of row
    // 16 w + L / 4, which holds chunk (L % 4) ^ qswz(row); with NJ = 1 waves 4..7 load
    // nothing into a sink past the tile.
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(w.qs, (uint64_t)N * (uint64_t)K / 2u);
    const bool qwave = wave < BN / 16;
    uint32_t qoff;
    {
        const int row = 16 * wave + (lane >> 2), c = (lane & 3) ^ qswz(row), n = n0 + row;
        qoff = qwave && n < N ? (uint32_t)n * (uint32_t)(K / 2) + (uint32_t)c * 16u : kOob;
    }
    const int qdst = qwave ? wave * 1024 : BN * 64;
    // Q6_K high bits: load t of wave w covers rows 16 w / (2 / NJ) + 8 t .. + 7 (32 bytes a
    // row), lane L dword L % 8 of row + L / 8.
    const __amdgpu_buffer_rsrc_t hr = make_rsrc(w.qh, FMT == Q6_K ? (uint64_t)N * (uint64_t)K / 4u : 0);
    uint32_t hoff[QHL > 0 ? QHL : 1];
#pragma unroll
    for (int t = 0; t < QHL; t++) {
        const int row = 8 * (QHL * wave + t) + (lane >> 3), n = n0 + row;
        hoff[t] = n < N ? (uint32_t)n * (uint32_t)(K / 4) + (uint32_t)(lane & 7) * 4u : kOob;
    }
    // Scale words: wave w loads those of rows RW w .. RW w + RW - 1 into its 256-byte slot.
    //  Q4_0: lane L < 2 RW: dword L % 2 (blocks 2 (L % 2), +1 of the stage) of row L / 2;
    //  Q4_K: lane L < 4 RW: dword L % 4 of row L / 4's 16-byte superblock record;
    //  Q6_K: lane L < 2 RW: dword L % 2 of row L / 2's eight int8 group scales of the stage;
    //        lane 32 + r (r < RW): the aligned dword holding row r's fp16 superblock d.
    //  (Q6_K's d section follows its sc section in the matrix's allocation, so one buffer
    //  resource from sc to the end of d's 256-byte-aligned section serves both.)
    const int nblk32 = K / 32, nsb = K / 256;
    const uint32_t d_rel = FMT == Q6_K ? (uint32_t)(w.d - w.sc) : 0u;
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(w.sc, FMT == Q4_0   ? (uint64_t)N * nblk32 * 2u
                        : FMT == Q4_K ? (uint64_t)N * nsb * 16u
                                      : (uint64_t)d_rel + align256((uint64_t)N * nsb * 2u));
    uint32_t soff = kOob, sstep = 0;
    bool s_is_d = false;
    {
        const int rbase = n0 + RW * wave;
        if (FMT == Q4_0) {
            const int n = rbase + (lane >> 1);
            if (lane < 2 * RW && n < N) soff = (uint32_t)n * (uint32_t)(nblk32 * 2) + (uint32_t)(lane & 1) * 4u;
            sstep = 8;
        } else if (FMT == Q4_K) {
            const int n = rbase + (lane >> 2);
            if (lane < 4 * RW && n < N) soff = (uint32_t)n * (uint32_t)(nsb * 16) + (uint32_t)(lane & 3) * 4u;
            sstep = 16;  // per superblock (two stages)
        } else {
            if (lane < 2 * RW) {
                const int n = rbase + (lane >> 1);
                if (n < N) soff = (uint32_t)n * (uint32_t)(K / 16) + (uint32_t)(lane & 1) * 4u;
                sstep = 8;
            } else if (lane >= 32 && lane < 32 + RW) {
                const int n = rbase + lane - 32;
                if (n < N) soff = d_rel + (uint32_t)n * (uint32_t)(nsb * 2);  // + 2 sb, rounded down to a dword
                s_is_d = true;
            }
        }
    }

    // Load p (0 <= p < P) of this wave for stage i.
    auto load = [&](int i, int p, uint8_t *xb, uint8_t *qb, uint8_t *hb, uint8_t *sb) {
        const int k0 = i * 128;
        const bool live = i < ns;
        if (p < XD) {
            const bool ok = live && k0 + xk[p] < K;
            dma16(xr, xb + (8 * p + wave) * 1024, ok ? xoff[p] : kOob, (uint32_t)k0 * 2u);
        } else if (p == XD) {
            dma16(qr, qb + qdst, live ? qoff : kOob, (uint32_t)i * 64u);
        } else if (p < XD + 1 + QHL) {
            const int t = p - XD - 1;
            dma4(hr, hb + (QHL * wave + t) * 256, live ? hoff[t] + (uint32_t)i * 32u : kOob);
        } else {
            uint32_t o = kOob;
            if (live && soff != kOob) {
                if (FMT == Q4_K) o = soff + (uint32_t)(i >> 1) * 16u;
                else if (FMT == Q6_K && s_is_d) o = (soff + (uint32_t)(i >> 1) * 2u) & ~3u;
                else o = soff + (uint32_t)i * sstep;
            }
            dma4(sr, sb + wave * 256, o);
        }
    };

    f32x4 acc[TM][NJ];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // B operand of column tile j, block c of stage i (lane group g: elements 8 g .. 8 g + 7).
    auto bop = [&](const uint8_t *qb, const uint8_t *hb, const uint8_t *sb, int i, int c, int j) -> bf16x8 {
        const int r = 16 * NJ * nw + 16 * j + m16;  // tile-relative W row
        const u32x2 q8 = *reinterpret_cast<const u32x2 *>(qb + r * 64 + ((c ^ qswz(r)) << 4) + 8 * (g & 1));
        const int sh = 4 * (g >> 1);
        uint32_t lo = (q8[0] >> sh) & 0x0F0F0F0Fu, hi = (q8[1] >> sh) & 0x0F0F0F0Fu;
        const uint8_t *slot = sb + (r / RW) * 256;
        const int rr = r % RW;
        if constexpr (FMT == Q4_0) {
            const float d = half_bits_to_float(*reinterpret_cast<const uint16_t *>(slot + rr * 8 + 2 * c));
            return deq8(lo, hi, d, -8.0f * d);
        } else if constexpr (FMT == Q4_K) {
            const u32x4 m = *reinterpret_cast<const u32x4 *>(slot + rr * 16);
            const int jsb = 4 * (i & 1) + c;
            const uint32_t sc = ((m[1] >> (4 * jsb)) & 15u) | (((m[3] >> (2 * jsb)) & 3u) << 4);
            const uint32_t mn = ((m[2] >> (4 * jsb)) & 15u) | (((m[3] >> (16 + 2 * jsb)) & 3u) << 4);
            const float d1 = half_bits_to_float(m[0] & 0xFFFFu) * (float)sc;
            const float m1 = half_bits_to_float(m[0] >> 16) * (float)mn;
            return deq8(lo, hi, d1, -m1);
        } else {
            const uint32_t h = *reinterpret_cast<const uint32_t *>(hb + r * 32 + (2 * c + (g & 1)) * 4);
            lo |= q6_high(h, sh);
            hi |= q6_high(h, 8 + sh);
            const int sc = (int)*reinterpret_cast<const int8_t *>(slot + rr * 8 + 2 * c + (g >> 1));
            const uint32_t dw = *reinterpret_cast<const uint32_t *>(slot + 128 + rr * 4);
            const int n = n0 + r;
            const uint32_t dbits = (((uint32_t)n * (uint32_t)nsb + (uint32_t)(i >> 1)) & 1u) ? dw >> 16 : dw & 0xFFFFu;
            const float ds = half_bits_to_float(dbits) * (float)sc;
            return deq8(lo, hi, ds, -32.0f * ds);
        }
    };

    // A operand of row tile t, block c: row 16 t + m16, chunk 4 c + g at slot chunk ^ m16.
    auto stage = [&](const uint8_t *xb, const uint8_t *qb, const uint8_t *hb, const uint8_t *sb, int i, uint8_t *xn,
                     uint8_t *qn, uint8_t *hn, uint8_t *sn) {
#pragma unroll
        for (int p = 0; p < P; p++) load(i + 2, p, xn, qn, hn, sn);
        // Block 0's W is dequantized before its MFMAs, block 1's between them, so the vector
        // ALU work of one block overlaps the matrix work of the other (both before the MFMAs,
        // the two waves of a SIMD dequantized in step with the matrix core idle). Every
        // accumulator's MFMAs keep their order, so results do not change.
        bf16x8 a[2][TM], b[2][NJ];
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const int c = 2 * bb + kh;
            const int ca = 4 * c + g;
            const int aoff = m16 * 256 + ((ca ^ m16) << 4);
#pragma unroll
            for (int t = 0; t < TM; t++) a[bb][t] = *reinterpret_cast<const bf16x8 *>(xb + t * 16 * 256 + aoff);
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) b[0][j] = bop(qb, hb, sb, i, kh, j);
        // block 1's column tile j is dequantized after block 0's MFMA number DQ (j + 1) - 1
        constexpr int DQ = TM * NJ / (NJ + 1) > 0 ? TM * NJ / (NJ + 1) : 1;
        int mi = 0;
#pragma unroll
        for (int bb = 0; bb < 2; bb++)
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[bb][t], b[bb][j], acc[t][j], 0, 0, 0);
                    if (bb == 0 && (mi + 1) % DQ == 0 && (mi + 1) / DQ <= NJ) {
                        const int jj = (mi + 1) / DQ - 1;
                        b[1][jj] = bop(qb, hb, sb, i, 2 + kh, jj);
                    }
                    mi++;
                }
    };

#pragma unroll
    for (int p = 0; p < P; p++) load(sbeg, p, xs0, qs0, hs0, ss0);
#pragma unroll
    for (int p = 0; p < P; p++) load(sbeg + 1, p, xs1, qs1, hs1, ss1);
    for (int i0 = sbeg; i0 < ns; i0 += 3) {
        wait_vm_lgkm0<P>();
        lds_barrier();
        stage(xs0, qs0, hs0, ss0, i0, xs2, qs2, hs2, ss2);
        wait_vm_lgkm0<P>();
        lds_barrier();
        stage(xs1, qs1, hs1, ss1, i0 + 1, xs0, qs0, hs0, ss0);
        wait_vm_lgkm0<P>();
        lds_barrier();
        stage(xs2, qs2, hs2, ss2, i0 + 2, xs1, qs1, hs1, ss1);
    }

    // ---- epilogue: the odd-block waves hand their partial tiles to the even-block waves,
    // which add them (even + odd) and store. Result element v of tile (t, j) is row
    // 16 t + 4 g + v, column 16 j + lane % 16 of the wave's columns.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float *const out = part ? part + (int64_t)blockIdx.y * M * N : y;
    float *red = reinterpret_cast<float *>(nw < 2 ? xs0 : xs1);
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < TM; t++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) red[((((nw & 1) * TM + t) * NJ + j) * 4 + v) * 64 + lane] = acc[t][j][v];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + 16 * t + 4 * g + v, col = n0 + 16 * NJ * nw + 16 * j + m16;
                const float s = acc[t][j][v] + red[((((nw & 1) * TM + t) * NJ + j) * 4 + v) * 64 + lane];
                if (row < M && col < N) out[(int64_t)row * N + col] = s;
            }
}

// y[i] = ((part[0][i] + part[1][i]) + ...) for i < n: the K splits' partial products added
// in split order (deterministic). A thread takes four consecutive elements when n % 4 == 0
// (every split then starts 16-byte aligned; y is), else one.
__global__ void __launch_bounds__(256)
sum_splits_kernel(const float *__restrict__ part, int splits, int64_t n, float *__restrict__ y) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    if (n % 4 == 0) {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n / 4; i += stride) {
            f32x4 v = reinterpret_cast<const f32x4 *>(part)[i];
            for (int r = 1; r < splits; r++) v += reinterpret_cast<const f32x4 *>(part + (int64_t)r * n)[i];
            reinterpret_cast<f32x4 *>(y)[i] = v;
        }
        return;
    }
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        float v = part[i];
        for (int r = 1; r < splits; r++) v += part[(int64_t)r * n + i];
        y[i] = v;
    }
}

}  // namespace gk
}  // namespace j4q

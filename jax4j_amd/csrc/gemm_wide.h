// Prefill GEMM, bf16 variant, register-staged (odd N at M >= 512): Y[M, N] = X[M, K] .
// bf16(W)[N, K]^T over Q8_0 weights, fp32 output.
//
// Tile BM x 64 NJ (BM = 64 or 128, NJ = 1 or 2) per workgroup of 8 waves, two waves per
// SIMD. K advances in stages of 64 (two Q8_0 blocks); wave w owns columns
// [16 NJ (w % 4), 16 NJ (w % 4 + 1)) of the tile and block w / 4 of every stage, for all BM
// rows: BM / 16 x NJ v_mfma_f32_16x16x32_bf16 accumulators. Each operand read from LDS
// feeds NJ MFMAs, so NJ = 2 halves the LDS reads per flop. The two waves that share
// columns (one per block of a stage) add their partial tiles through LDS at the end, in a
// fixed order.
//
// What bounds it is the rate at which a CU's vector memory path accepts cache lines (about
// one 128-byte line per 4 clocks, measured): every load instruction here touches only whole
// lines, 8 per instruction.
//  - X (bf16, rows 8 KB apart for K = 4096): BM rows x 128 bytes per stage, 8 rows per
//    load instruction, stored with 128-bit writes into three LDS stage buffers of 128-byte
//    rows whose 16-byte chunks are XOR-swizzled by the row (chunk c of row r at
//    c ^ ((r / 2) % 8)): the LDS serves 16 lanes of a 128-bit access per cycle from 64
//    banks, and the 16 rows of an MFMA operand read then fall on distinct banks.
//  - W int8: 128 bytes (four blocks, two stages) of each of the tile's rows per load, 8 rows
//    per instruction, into an LDS buffer with rows padded to 144 bytes; each wave reads its
//    8 bytes per lane from there and dequantizes them in registers to bf16(d * q) (d * q is
//    exact in fp32, the conversion rounds to nearest even).
//  - W scales from the block-major copy of the Q8_0 split layout: the 16 rows of an operand
//    tile read one contiguous 32-byte run per block.
//  - MFMA lane group g = lane / 16 supplies k = 8 g + 0..7 of its block, for A (X) and B (W)
//    alike.
// Pipeline, one barrier per stage: global loads run R stages ahead in a ring of register
// sets; X of stage i + 2 (and W of its stage pair) is stored into LDS while the MFMA
// operands of stage i + 1 are read and the MFMAs of stage i run on operands read one
// iteration earlier, so LDS traffic and matrix work overlap. A buffer is rewritten only
// after every wave passed the barrier that follows its last read. The ring has no branch:
// the stages past the end (at most R - 1) load zeros and add exact zeros, which keeps the
// compiler's memory-counter waits exact.
#pragma once

#include "j4q_common.h"

namespace j4q {
namespace gw {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr uint32_t kOob = 0x80000000u;
constexpr int kWRow = 144;             // W LDS row: 128 bytes (two stages) + 16 bytes of padding

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint64_t bytes) {
    const uint32_t n = bytes > 0x7fffffffull ? 0x7fffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, 0x00020000);
}

// bf16(d * q) of the 8 int8 in q, packed as an MFMA operand.
__device__ __forceinline__ bf16x8 dequant8(u32x2 q, float d) {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t v = q[j];
        const float f0 = d * (float)(int8_t)(v & 0xFFu), f1 = d * (float)(int8_t)((v >> 8) & 0xFFu);
        const float f2 = d * (float)(int8_t)((v >> 16) & 0xFFu), f3 = d * (float)(int8_t)(v >> 24);
        o[2 * j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{f0, f1}), bf16x2));
        o[2 * j + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{f2, f3}), bf16x2));
    }
    return __builtin_bit_cast(bf16x8, o);
}

// grid = ceil(M / BM) * ceil(N / (64 NJ)) workgroups of 512 threads. Requires K % 32 == 0,
// M * K * 2 < 2^31, N * K < 2^31 and the block-major scale copy in w.d.
template <int BM, int NJ, int R>
__global__ void __launch_bounds__(512)
gemm_bf16_wide(QMat w, const uint16_t *__restrict__ x, float *__restrict__ y, int M) {
    static_assert(R % 2 == 0 && R >= 4, "the ring unrolls by an even R of at least 4");
    static_assert(BM == 64 || BM == 128, "64 or 128 rows");
    constexpr int BN = 64 * NJ, TM = BM / 16, XC = BM / 64;  // row tiles, X chunks per thread
    constexpr int kStageBytes = BM * 128;                     // X: 64 bf16 of k per row
    constexpr int kWBuf = BN * kWRow;
    constexpr int kXRegion = 3 * kStageBytes;
    constexpr int kRedBytes = 4 * TM * NJ * 4 * 64 * 4;  // partial tiles of the 4 second-block waves
    constexpr int kLds = kXRegion + 2 * kWBuf > kRedBytes ? kXRegion + 2 * kWBuf : kRedBytes;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32, ns = (K + 63) / 64;
    const int mt = (M + BM - 1) / BM;
    // Workgroup b runs on XCD b % 8; tile order is m fastest and each XCD takes a contiguous
    // range of it, so the m tiles of a group of n tiles (the same W rows) share an L2.
    const int total = (int)gridDim.x;
    int tile = (int)blockIdx.x;
    if (total % 8 == 0) tile = (tile % 8) * (total / 8) + tile / 8;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = wave & 3, kh = wave >> 2;  // column group, block of the stage
    const int m16 = lane & 15, g = lane >> 4;

    // X: thread t stages chunks q = t + 512 j (row q / 8, 16-byte chunk q % 8) of a stage.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint64_t)M * (uint64_t)K * 2u);
    uint32_t xoff[XC];
    int xk[XC], xlds[XC];
#pragma unroll
    for (int j = 0; j < XC; j++) {
        const int q = tid + 512 * j, row = q >> 3, c = q & 7, gm = m0 + row;
        xoff[j] = gm < M ? (uint32_t)gm * (uint32_t)K * 2u + (uint32_t)c * 16u : kOob;
        xk[j] = c * 8;
        xlds[j] = row * 128 + ((c ^ ((row >> 1) & 7)) << 4);
    }
    // W bytes: thread t stages chunks q = t + 512 j (tile row q / 8, 16-byte chunk q % 8) of
    // the 128 bytes a stage pair covers.
    const __amdgpu_buffer_rsrc_t wq = make_rsrc(w.qs, (uint64_t)N * (uint64_t)K);
    uint32_t woff[NJ];
    int wk[NJ], wlds[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int q = tid + 512 * j, row = q >> 3, c = q & 7, n = n0 + row;
        woff[j] = n < N ? (uint32_t)n * (uint32_t)K + (uint32_t)c * 16u : kOob;
        wk[j] = c * 16;
        wlds[j] = row * kWRow + c * 16;
    }
    // W scales: lane (row 16 j + lane % 16 of the wave's columns) reads the scale of block
    // kh of the stage from the block-major copy.
    const __amdgpu_buffer_rsrc_t wd = make_rsrc(w.d, (uint64_t)N * (uint64_t)nblk * 2u);
    uint32_t doff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int n = n0 + 16 * NJ * nw + 16 * j + m16;
        doff[j] = n < N ? (uint32_t)n * 2u : kOob;
    }

    struct Set {
        u32x4 x[XC];
        u32x4 q[NJ];  // loaded with even stages only: the stage pair's W bytes
        uint32_t d[NJ];
    };
    Set set[R];
    // Stage i covers k [64 i, 64 i + 64); stages at or past ns (and blocks past the row)
    // load nothing.
    auto load = [&](int i, Set &S_, bool pair) {
        const bool live = i < ns;
        const int k0 = i * 64;
#pragma unroll
        for (int j = 0; j < XC; j++) {
            const bool ok = live && k0 + xk[j] < K;
            S_.x[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xoff[j] : kOob, (uint32_t)k0 * 2u, 0));
        }
        if (pair) {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const bool ok = live && k0 + wk[j] < K;
                S_.q[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wq, ok ? woff[j] : kOob, (uint32_t)k0, 0));
            }
        }
        const int kb = 2 * i + kh;  // this wave's block (wave-uniform)
        const bool bok = live && kb < nblk;
#pragma unroll
        for (int j = 0; j < NJ; j++)
            S_.d[j] = __builtin_amdgcn_raw_buffer_load_b16(wd, doff[j], bok ? (uint32_t)kb * (uint32_t)N * 2u : kOob, 0);
    };

    f32x4 acc[TM][NJ];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 bfr[2][NJ];  // B operands of a stage, double-buffered

    uint8_t *const xbase = lds;
    uint8_t *const wbase = lds + kXRegion;
    auto store_x = [&](const Set &S_, int buf) {
#pragma unroll
        for (int j = 0; j < XC; j++) *reinterpret_cast<u32x4 *>(&xbase[buf * kStageBytes + xlds[j]]) = S_.x[j];
    };
    auto store_w = [&](const Set &S_, int wbuf) {
#pragma unroll
        for (int j = 0; j < NJ; j++) *reinterpret_cast<u32x4 *>(&wbase[wbuf * kWBuf + wlds[j]]) = S_.q[j];
    };
    // B operand bytes of stage i for column tile j: row 16 NJ nw + 16 j + lane % 16, bytes
    // 32 (2 (i % 2) + kh) + 8 g of the stage pair's 128.
    const int wrd = (16 * NJ * nw + m16) * kWRow + 32 * kh + 8 * g;
    auto read_w = [&](int wbuf, int odd, u32x2 (&wb)[NJ]) {
#pragma unroll
        for (int j = 0; j < NJ; j++) wb[j] = *reinterpret_cast<const u32x2 *>(&wbase[wbuf * kWBuf + wrd + 16 * j * kWRow + 64 * odd]);
    };
    // A operand of row tile t: row 16 t + lane % 16, chunk 4 kh + g (the swizzle term
    // (row / 2) % 8 does not depend on t).
    const int aoff = m16 * 128 + (((4 * kh + g) ^ ((m16 >> 1) & 7)) << 4);
    auto read_a = [&](int buf, bf16x8 (&a)[TM]) {
#pragma unroll
        for (int t = 0; t < TM; t++) a[t] = *reinterpret_cast<const bf16x8 *>(&xbase[buf * kStageBytes + t * 16 * 128 + aoff]);
    };

    // Prologue: stages 0 .. R-1 in flight; X of stages 0 and 1 and W of pair 0 in LDS; the
    // operands of stage 0 read and dequantized.
#pragma unroll
    for (int r = 0; r < R; r++) {
        load(r, set[r], (r & 1) == 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    bf16x8 a[2][TM];
    u32x2 wb[NJ];
    store_x(set[0], 0);
    store_x(set[1], 1);
    store_w(set[0], 0);
    __syncthreads();
    read_a(0, a[0]);
    read_w(0, 0, wb);
#pragma unroll
    for (int j = 0; j < NJ; j++) bfr[0][j] = dequant8(wb[j], half_bits_to_float(set[0].d[j]));
    // Iteration i (set i % R, X buffer i % 3, W buffer (i / 2) % 2): the barrier publishes X
    // of stage i + 1 (and W of its pair) and frees the buffers of stage i - 1; then the loads
    // of stage i + R, the operand reads of stage i + 1, the stores of stage i + 2, the
    // dequantization of stage i + 1 and the MFMAs of stage i.
    int b0 = 0;  // i % 3
    for (int i0 = 0; i0 < ns; i0 += R) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            // i0 is a multiple of the even R, so i % 2 == r % 2
            const int i = i0 + r;
            const int b1 = b0 == 2 ? 0 : b0 + 1, b2 = b1 == 2 ? 0 : b1 + 1;
            __syncthreads();
            load(i + R, set[r], (r & 1) == 0);
            __builtin_amdgcn_sched_barrier(0);
            // the LDS traffic goes first: the wait before the next barrier then finds it done
            read_a(b1, a[(r + 1) & 1]);
            read_w(((i + 1) >> 1) & 1, (r + 1) & 1, wb);
            store_x(set[(r + 2) % R], b2);
            if ((r & 1) == 0) store_w(set[(r + 2) % R], ((i + 2) >> 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NJ; j++) bfr[(r + 1) & 1][j] = dequant8(wb[j], half_bits_to_float(set[(r + 1) % R].d[j]));
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r & 1][t], bfr[r & 1][j], acc[t][j], 0, 0, 0);
            b0 = b1;
        }
    }

    // ---- epilogue: the second-block waves hand their partial tiles to the first-block
    // waves, which add them (first + second) and store. Result element v of tile (t, j) is
    // row 16 t + 4 g + v, column 16 j + lane % 16 of the wave's columns.
    float *red = reinterpret_cast<float *>(lds);
    __syncthreads();  // every wave is past its last read of the stage buffers
    if (kh == 1) {
#pragma unroll
        for (int t = 0; t < TM; t++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) red[(((nw * TM + t) * NJ + j) * 4 + v) * 64 + lane] = acc[t][j][v];
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
                const float s = acc[t][j][v] + red[(((nw * TM + t) * NJ + j) * 4 + v) * 64 + lane];
                if (row < M && col < N) y[(int64_t)row * N + col] = s;
            }
}

// ---- The same product with the tiles loaded straight into LDS ----------------------------
//
// buffer_load_dwordx4 ... lds writes a wave's 64 x 16 bytes to LDS at M0 + 16 lane without
// passing through VGPRs (lane layout and zero fill of out-of-range lanes checked on MI355X).
// The host pass of hipcc checks the builtin's 16-byte size against the host target and
// rejects it, so the call exists in the device pass only.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t vo, uint32_t so) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, vo, so, 0, 0);
#endif
}

__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t vo) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4, vo, 0, 0, 0);
}

__device__ __forceinline__ void dma4s(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t vo, uint32_t so) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4, vo, so, 0, 0);
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding; expcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

// A workgroup barrier without __syncthreads()'s release fence: the fence would wait for every
// LDS load in flight (vmcnt(0)), which is the ring this kernel keeps open. The empty asm
// statements keep the compiler from moving memory accesses across it.
// Wave priority p (0..3; s_setprio takes an immediate, so p must fold to a constant). The
// stage loops below lower a wave's priority as it gets through a stage, so the wave of a SIMD
// that is behind issues first and the two reach the next barrier together (A/B pairs on one
// box, three rounds, bench with the quantizer: int8 M = 512 36.2-38.2 -> 35.5-36.9 us, M = 2048
// 132.5-133.6 -> 129.9-131.1 us; bf16 M = 2048 97.7-102.2 -> 97.4-98.7 us, M = 512 level).
__device__ __forceinline__ void wave_prio(int p) {
    if (p >= 3) __builtin_amdgcn_s_setprio(3);
    else if (p == 2) __builtin_amdgcn_s_setprio(2);
    else if (p == 1) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// W-tile swizzle of gemm_bf16_lds: 16-byte chunk c of row r sits at slot c ^ wswz(r). Bits
// 1..3 of the row spread the 16 rows of one operand read over all banks; bit 4 moves rows 16
// apart by 64 bytes, so a wave's reads of two column tiles (rows r and r + 16) never share
// banks and never sit a constant offset apart (the compiler merged those into one
// ds_read2st64_b64 whose two halves conflicted: 2.2 M bank-conflict cycles per 128 x 128
// launch at M = 2048).
__device__ __forceinline__ int wswz(int row) { return ((row >> 1) & 7) ^ (((row >> 4) & 1) << 2); }

// Prefill GEMM, bf16 variant for even N from M = 65 on (whenever its grid has at least 128
// workgroups; launch_gemm_q8_bf16 in gemm.hip picks the tile), results bit-identical to
// gemm_bf16_wide (the same blocks go to the same waves in the same order):
//  - Tile BM x 64 NJ per workgroup of 8 waves; wave w owns columns [16 NJ (w % 4), +16 NJ)
//    and blocks 2 b + w / 4 (b = 0, 1) of every 128-k stage, for all BM rows.
//  - Every stage moves straight from global memory into one of three LDS stage buffers:
//    X as BM rows x 256 bytes (16-byte chunk c of row r at c ^ (r % 16): the 16 rows of an
//    operand read fall on distinct banks), W as BN rows x 128 bytes (chunk c of row r at
//    c ^ wswz(r)), and each wave's scales of the stage into its own 256-byte slot.
//    Each wave's LDS loads pick the global chunk that belongs at their lane's LDS slot.
//  - The buffers are separate __shared__ arrays and the ring is unrolled by three, so the
//    compiler knows which loads write the buffer a read touches and adds no waits of its
//    own; the kernel waits for its stage with vmcnt(loads of one stage) and a barrier.
//  - Iteration i: wait for own stage-i loads and LDS reads, barrier (stage i is in LDS for
//    every wave, every read of stage i - 1 is done), load stage i + 2 into the buffers of
//    stage i - 1, read all operands of stage i, dequantize W and run the MFMAs. With ILV
//    the stage i + 2 loads are spread between the MFMAs (measured faster at 128 x 128
//    tiles: a wave blocks while the load path accepts its loads); otherwise they go first.
//  - Stages past the end load zeros (out-of-range offsets) and add exact zeros; all LDS
//    loads have landed (vmcnt(0)) before the partial tiles reuse the X buffers.
// grid = ceil(M / BM) * ceil(N / (64 NJ)) workgroups of 512 threads. Requires N even,
// K % 32 == 0, M * K * 2 < 2^31, N * K < 2^31 and the block-major scale copy in w.d.
template <int BM, int NJ, bool ILV>
__global__ void __launch_bounds__(512)
gemm_bf16_lds(QMat w, const uint16_t *__restrict__ x, float *__restrict__ y, int M) {
    static_assert(BM == 64 || BM == 128, "64 or 128 rows");
    constexpr int BN = 64 * NJ, TM = BM / 16, XD = BM / 32;  // X loads per wave and stage
    constexpr int kX = BM * 256, kW = BN * 128;
    constexpr int P = XD + NJ + 1;  // vector-memory instructions per wave and stage
    __shared__ __attribute__((aligned(1024))) uint8_t xs0[kX], xs1[kX], xs2[kX];
    __shared__ __attribute__((aligned(1024))) uint8_t ws0[kW], ws1[kW], ws2[kW];
    __shared__ __attribute__((aligned(1024))) uint8_t ds0[2048], ds1[2048], ds2[2048];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32, ns = (K + 127) / 128;
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
    // W load j covers rows 8 (8 j + wave) .. +7; slot L % 8 of row 8 (8 j + wave) + L / 8
    // holds chunk (L % 8) ^ wswz(row).
    const __amdgpu_buffer_rsrc_t wq = make_rsrc(w.qs, (uint64_t)N * (uint64_t)K);
    uint32_t woff[NJ];
    int wk[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int row = 8 * (8 * j + wave) + (lane >> 3), c = (lane & 7) ^ wswz(row), n = n0 + row;
        woff[j] = n < N ? (uint32_t)n * (uint32_t)K + (uint32_t)c * 16u : kOob;
        wk[j] = c * 16;
    }
    // Scales, 4 bytes per lane: lane L < 16 NJ loads the scales of rows r + 2 (L % 8 NJ) and
    // r + 2 (L % 8 NJ) + 1 (r = the wave's first column) for block 2 (L / 8 NJ) + kh of the
    // stage; the slot is [2 blocks][16 NJ rows] fp16 (N even keeps both rows in range).
    const __amdgpu_buffer_rsrc_t wd = make_rsrc(w.d, (uint64_t)N * (uint64_t)nblk * 2u);
    const int dbb = lane / (8 * NJ), drow = n0 + 16 * NJ * nw + 2 * (lane % (8 * NJ));
    const bool dlane = lane < 16 * NJ && drow < N;
    const uint32_t doff = (uint32_t)drow * 2u;

    // Load p (0 <= p < P) of this wave for stage i.
    auto load = [&](int i, int p, uint8_t *xb, uint8_t *wb, uint8_t *db) {
        const int k0 = i * 128;
        const bool live = i < ns;
        if (p < XD) {
            const bool ok = live && k0 + xk[p] < K;
            dma16(xr, xb + (8 * p + wave) * 1024, ok ? xoff[p] : kOob, (uint32_t)k0 * 2u);
        } else if (p < XD + NJ) {
            const int j = p - XD;
            const bool ok = live && k0 + wk[j] < K;
            dma16(wq, wb + (8 * j + wave) * 1024, ok ? woff[j] : kOob, (uint32_t)k0);
        } else {
            const int kb = 4 * i + 2 * dbb + kh;
            const bool ok = live && dlane && kb < nblk;
            dma4(wd, db + wave * 256, ok ? doff + (uint32_t)kb * (uint32_t)N * 2u : kOob);
        }
    };

    f32x4 acc[TM][NJ];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Stage in (xb, wb, db) and the loads of stage inext into (xn, wn, dn).
    // A operand of row tile t, block b: row 16 t + m16, chunk 4 (2 b + kh) + g, at slot
    // chunk ^ m16. B operand of column tile j: row 16 NJ nw + 16 j + m16, bytes
    // 32 (2 b + kh) + 8 g, i.e. chunk 2 (2 b + kh) + g / 2 at slot chunk ^ wswz(row), half
    // g % 2.
    auto stage = [&](const uint8_t *xb, const uint8_t *wb, const uint8_t *db, int inext, uint8_t *xn, uint8_t *wn,
                     uint8_t *dn) {
        if (!ILV) {
#pragma unroll
            for (int p = 0; p < P; p++) load(inext, p, xn, wn, dn);
        }
        // Operands of the stage's two blocks (bb = 0, 1). Block 0's W is dequantized before
        // its MFMAs; block 1's operands are read right behind it, and its W is dequantized
        // between block 0's MFMAs, so the vector ALU work of one block overlaps the matrix
        // work of the other (all at once before the MFMAs, the two waves of a SIMD dequantized
        // in step and left the matrix core idle meanwhile). The MFMAs of every accumulator run
        // in the same order as before, so results do not change.
        bf16x8 a[2][TM], b[2][NJ];
        u32x2 q1[NJ];
        uint32_t d1[NJ];
        auto read_block = [&](int bb, u32x2 (&q)[NJ], uint32_t (&d)[NJ]) {
            const int ca = 4 * (2 * bb + kh) + g;
            const int aoff = m16 * 256 + ((ca ^ m16) << 4);
#pragma unroll
            for (int t = 0; t < TM; t++) a[bb][t] = *reinterpret_cast<const bf16x8 *>(xb + t * 16 * 256 + aoff);
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int row = 16 * NJ * nw + 16 * j + m16, cb = 2 * (2 * bb + kh) + (g >> 1);
                q[j] = *reinterpret_cast<const u32x2 *>(wb + row * 128 + ((cb ^ wswz(row)) << 4) + 8 * (g & 1));
                d[j] = *reinterpret_cast<const uint16_t *>(db + wave * 256 + (bb * 16 * NJ + 16 * j + m16) * 2);
            }
        };
        wave_prio(1);
        {
            u32x2 q0[NJ];
            uint32_t d0[NJ];
            read_block(0, q0, d0);
#pragma unroll
            for (int j = 0; j < NJ; j++) b[0][j] = dequant8(q0[j], half_bits_to_float(d0[j]));
        }
        read_block(1, q1, d1);
        constexpr int NM = 2 * TM * NJ, STRIDE = NM / P > 0 ? NM / P : 1;
        // block 1's column tile j is dequantized after block 0's MFMA number DQ (j + 1) - 1
        constexpr int DQ = TM * NJ / (NJ + 1) > 0 ? TM * NJ / (NJ + 1) : 1;
        int mi = 0, p = 0;
#pragma unroll
        for (int bb = 0; bb < 2; bb++)
#pragma unroll
            for (int t = 0; t < TM; t++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    if (bb == 1 && t == 0 && j == 0) wave_prio(0);  // on to the stage's second block
                    acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[bb][t], b[bb][j], acc[t][j], 0, 0, 0);
                    if (ILV && mi % STRIDE == STRIDE - 1 && p < P) {
                        __builtin_amdgcn_sched_barrier(0);
                        load(inext, p, xn, wn, dn);
                        __builtin_amdgcn_sched_barrier(0);
                        p++;
                    }
                    if (bb == 0 && (mi + 1) % DQ == 0 && (mi + 1) / DQ <= NJ) {
                        const int jj = (mi + 1) / DQ - 1;
                        b[1][jj] = dequant8(q1[jj], half_bits_to_float(d1[jj]));
                    }
                    mi++;
                }
        if (ILV) {
#pragma unroll
            for (; p < P; p++) load(inext, p, xn, wn, dn);
        }
    };

#pragma unroll
    for (int p = 0; p < P; p++) load(0, p, xs0, ws0, ds0);
#pragma unroll
    for (int p = 0; p < P; p++) load(1, p, xs1, ws1, ds1);
    for (int i0 = 0; i0 < ns; i0 += 3) {
        wait_vm_lgkm0<P>();
        lds_barrier();
        stage(xs0, ws0, ds0, i0 + 2, xs2, ws2, ds2);
        wait_vm_lgkm0<P>();
        lds_barrier();
        stage(xs1, ws1, ds1, i0 + 3, xs0, ws0, ds0);
        wait_vm_lgkm0<P>();
        lds_barrier();
        stage(xs2, ws2, ds2, i0 + 4, xs1, ws1, ds1);
    }

    // ---- epilogue: the odd-block waves hand their partial tiles to the even-block waves,
    // which add them (even + odd) and store. Result element v of tile (t, j) is row
    // 16 t + 4 g + v, column 16 j + lane % 16 of the wave's columns.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
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
                if (row < M && col < N) y[(int64_t)row * N + col] = s;
            }
}

}  // namespace gw
}  // namespace j4q

namespace j4q {
namespace gw {

// Prefill GEMM, bf16 variant for small M (M <= 128): the weights are the traffic (17.8 MB
// for N = K = 4096), so every CU streams its own 16 rows of W once over all of K, for all
// BM rows of X (BM = 32, 64 or 128): grid = ceil(M / BM) * ceil(N / 16) workgroups of 8
// waves. K advances in stages of 256 KPW (8 KPW Q8_0 blocks); wave w takes blocks w, w + 8,
// ... of every stage: BM / 16 v_mfma_f32_16x16x32_bf16 accumulators of 16 columns. The 8
// waves' partial tiles are added through LDS at the end in wave order (deterministic).
//  - X: BM rows x 512 KPW bytes per stage through two LDS buffers, whole-line loads,
//    16-byte chunk c of row r stored at chunk c ^ (r % 16): the 16 rows of an operand read
//    fall on distinct banks.
//  - W: 16 rows x 256 KPW bytes per stage through two LDS buffers of rows padded by 16
//    bytes; each wave reads 8 bytes per lane of each of its blocks and dequantizes them to
//    bf16(d * q) in registers, with d from the block-major scale copy.
// One barrier per stage; global loads run R stages ahead in a ring of register sets; stages
// past the end load zeros and add exact zeros.
template <int BM, int KPW, int R>
__global__ void __launch_bounds__(512)
gemm_bf16_narrow(QMat w, const uint16_t *__restrict__ x, float *__restrict__ y, int M) {
    static_assert(BM == 32 || BM == 64 || BM == 128, "32, 64 or 128 rows");
    static_assert(KPW == 1 || KPW == 2, "one or two blocks per wave and stage");
    static_assert(R % 2 == 0 && R >= 2, "the ring unrolls by an even R");
    constexpr int TM = BM / 16, XC = BM * KPW / 16;  // row tiles; X chunks per thread and stage
    constexpr int SK = 256 * KPW, XROW = 2 * SK, WROW = SK + 16;
    constexpr int kXStage = BM * XROW, kWStage = 16 * WROW;
    constexpr int kRed = 7 * TM * 4 * 64 * 4;  // partial tiles of waves 1..7
    constexpr int kLds = 2 * kXStage + 2 * kWStage > kRed ? 2 * kXStage + 2 * kWStage : kRed;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32, ns = (K + SK - 1) / SK;
    const int mt = (M + BM - 1) / BM;
    // Workgroup b runs on XCD b % 8: each XCD takes a contiguous range of tiles (m fastest).
    const int total = (int)gridDim.x;
    int tile = (int)blockIdx.x;
    if (total % 8 == 0) tile = (tile % 8) * (total / 8) + tile / 8;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * 16;

    const int tid = (int)threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m16 = lane & 15, g = lane >> 4;

    // X: thread t stages chunks q = t + 512 j (row q / (32 KPW), 16-byte chunk q % (32 KPW)).
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint64_t)M * (uint64_t)K * 2u);
    uint32_t xoff[XC];
    int xk[XC], xlds[XC];
#pragma unroll
    for (int j = 0; j < XC; j++) {
        const int q = tid + 512 * j, row = q / (32 * KPW), c = q % (32 * KPW), gm = m0 + row;
        xoff[j] = gm < M ? (uint32_t)gm * (uint32_t)K * 2u + (uint32_t)c * 16u : kOob;
        xk[j] = c * 8;
        xlds[j] = row * XROW + ((c ^ (row & 15)) << 4);
    }
    // W: thread t < 256 KPW stages chunk t (row t / (16 KPW), 16-byte chunk t % (16 KPW)) of
    // the stage's bytes of each row; the other threads load nothing.
    const __amdgpu_buffer_rsrc_t wq = make_rsrc(w.qs, (uint64_t)N * (uint64_t)K);
    const bool wthr = tid < 256 * KPW;
    const int wrow = (tid / (16 * KPW)) & 15, wc = tid % (16 * KPW), wn = n0 + wrow;
    const uint32_t woff = (wthr && wn < N) ? (uint32_t)wn * (uint32_t)K + (uint32_t)wc * 16u : kOob;
    const int wlds = wrow * WROW + wc * 16;
    const __amdgpu_buffer_rsrc_t wd = make_rsrc(w.d, (uint64_t)N * (uint64_t)nblk * 2u);
    const uint32_t doff = n0 + m16 < N ? (uint32_t)(n0 + m16) * 2u : kOob;

    struct Set {
        u32x4 x[XC];
        u32x4 q;
        uint32_t d[KPW];
    };
    Set set[R];
    auto load = [&](int i, Set &S_) {
        const bool live = i < ns;
        const int k0 = i * SK;
#pragma unroll
        for (int j = 0; j < XC; j++) {
            const bool ok = live && k0 + xk[j] < K;
            S_.x[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xoff[j] : kOob, (uint32_t)k0 * 2u, 0));
        }
        const bool wok = live && k0 + wc * 16 < K;
        S_.q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wq, wok ? woff : kOob, (uint32_t)k0, 0));
#pragma unroll
        for (int j = 0; j < KPW; j++) {
            const int kb = 8 * KPW * i + 8 * j + wave;  // this wave's blocks (wave-uniform)
            S_.d[j] = __builtin_amdgcn_raw_buffer_load_b16(wd, doff, live && kb < nblk ? (uint32_t)kb * (uint32_t)N * 2u : kOob, 0);
        }
    };
    uint8_t *const xbase = lds;
    uint8_t *const wbase = lds + 2 * kXStage;
    auto store = [&](const Set &S_, int buf) {
#pragma unroll
        for (int j = 0; j < XC; j++) *reinterpret_cast<u32x4 *>(&xbase[buf * kXStage + xlds[j]]) = S_.x[j];
        if (wthr) *reinterpret_cast<u32x4 *>(&wbase[buf * kWStage + wlds]) = S_.q;
    };
    // A operand of row tile t, block j: row 16 t + lane % 16, chunk 4 (8 j + wave) + g.
    int aoff[KPW], boff[KPW];
#pragma unroll
    for (int j = 0; j < KPW; j++) {
        aoff[j] = m16 * XROW + (((4 * (8 * j + wave) + g) ^ m16) << 4);
        boff[j] = m16 * WROW + 32 * (8 * j + wave) + 8 * g;
    }

    f32x4 acc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int r = 0; r < R; r++) {
        load(r, set[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
    store(set[0], 0);
    // Iteration i: the barrier publishes stage i (stored during iteration i - 1) and frees
    // the other buffers (their last reader, stage i - 1, is done); the loads of stage i + R
    // go into the set stage i used; stage i + 1 is stored while stage i is multiplied.
    for (int i0 = 0; i0 < ns; i0 += R) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = i0 + r;  // i0 is a multiple of the even R: buffer i % 2 == r % 2
            __syncthreads();
            bf16x8 a[KPW][TM];
            u32x2 wb[KPW];
            float d[KPW];
#pragma unroll
            for (int j = 0; j < KPW; j++) {
#pragma unroll
                for (int t = 0; t < TM; t++) a[j][t] = *reinterpret_cast<const bf16x8 *>(&xbase[(r & 1) * kXStage + t * 16 * XROW + aoff[j]]);
                wb[j] = *reinterpret_cast<const u32x2 *>(&wbase[(r & 1) * kWStage + boff[j]]);
                d[j] = half_bits_to_float(set[r].d[j]);
            }
            load(i + R, set[r]);
            __builtin_amdgcn_sched_barrier(0);
            store(set[(r + 1) % R], (r + 1) & 1);
#pragma unroll
            for (int j = 0; j < KPW; j++) {
                const bf16x8 b = dequant8(wb[j], d[j]);
#pragma unroll
                for (int t = 0; t < TM; t++) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j][t], b, acc[t], 0, 0, 0);
            }
        }
    }

    // ---- epilogue: waves 1..7 hand their partial tiles to wave 0, which adds them in wave
    // order and stores. Result element v of row tile t is row 16 t + 4 g + v, column
    // lane % 16.
    float *red = reinterpret_cast<float *>(lds);
    __syncthreads();
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < TM; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) red[(((wave - 1) * TM + t) * 4 + v) * 64 + lane] = acc[t][v];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float s = acc[t][v];
            for (int ww = 0; ww < 7; ww++) s += red[((ww * TM + t) * 4 + v) * 64 + lane];
            const int row = m0 + 16 * t + 4 * g + v, col = n0 + m16;
            if (row < M && col < N) y[(int64_t)row * N + col] = s;
        }
}

}  // namespace gw
}  // namespace j4q

namespace j4q {
namespace gw {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));

// Int8 variant of the prefill GEMM: Y[m, n] = sum over blocks b, in block order, of
// fma(float(I_b[m, n]), fl(sx[m, b] * dw[n, b]), acc) with I_b the exact int32 dot of the
// quantized activations and the Q8_0 quants of block b; every output is folded by one lane
// (over all of K, or over each of a few contiguous K ranges whose partials are then added in
// order), so results are bit-identical to a sequential fp32 loop over the blocks (the
// oracle's emulation). The scale products fl(sx * dw) come from the matrix core as outer
// products in the int8 product's layout, so the vector ALU does two operations per output
// and block (convert, FMA). Kernels: gemm_i8_small (M <= 256) and gemm_i8_lds (above).

}  // namespace gw
}  // namespace j4q

namespace j4q {
namespace gw {

typedef int32_t i32x4s __attribute__((ext_vector_type(4)));

// Prefill GEMM, int8 variant for small M: the fold above on 16 x 32 tiles, with K
// cut into RG = 1 or 4 contiguous ranges of whole stages, each run by its own pair of waves
// through its own LDS buffers. With one lane per output over all of K, M = 32 would have only
// 512 16 x 16 tiles (two waves per CU) whose 32 stages run back to back; four ranges give
// eight waves per workgroup and a quarter of the stages each (used while the tiles do not
// exceed the CUs; with more tiles the single range is faster: M = 128 27.4 us against 42.6). Wave (p, h) = (w / 2, w % 2) owns
// columns 16 h .. 16 h + 15 and range p (stages [p L, (p + 1) L), L = ceil(stages / 4)), one
// v_mfma_i32_16x16x32_i8 per block (operand lane (r, g): row r % 16, 8 bytes of k at 8 g),
// folded in block order into its partial; the partials meet at the end as
// ((p0 + p1) + p2) + p3, the association of the oracle's emulation with four ranges.
// Stages of four blocks (one 128-byte line per row) go through two LDS buffers per range
// with 16-byte chunk c of row r at chunk c ^ ((r / 2) % 8) of 128-byte rows (the 16 rows of an
// operand read fall on distinct banks); a stage's four MFMAs are issued before their folds.
// Every range runs the same number of iterations (its stages past its range load nothing
// and compute nothing), so all waves meet at every barrier. Requires K % 32 == 0,
// N % 8 == 0, M * K < 2^31 and N * K < 2^31.
template <int R, int RG>
__global__ void __launch_bounds__(128 * RG)
gemm_i8_small(QMat w, const int8_t *__restrict__ xq, const float *__restrict__ xs, float *__restrict__ y, int M) {
    static_assert(R % 2 == 0 && R >= 2, "the ring unrolls by an even R");
    constexpr int BM = 16, BN = 32, SB = 4;  // rows, columns, blocks per stage
    constexpr int kXS = BM * 128, kWS = BN * 128, kSxS = SB * BM * 4, kDwS = SB * BN * 4;
    constexpr int kBuf = kXS + kWS + kSxS + kDwS;
    static_assert(RG == 1 || RG == 4, "one or four K ranges");
    static_assert((RG - 1) * 2 * 64 * 16 <= 2 * kBuf, "partials fit one range's buffers");
    __shared__ __attribute__((aligned(16))) uint8_t lds_all[RG * 2 * kBuf];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32, nst = (nblk + SB - 1) / SB;
    const int L = (nst + RG - 1) / RG;  // stages per range
    const int mt = (M + BM - 1) / BM;
    const int total = (int)gridDim.x;
    int tile = (int)blockIdx.x;
    if (total % 8 == 0) tile = (tile % 8) * (total / 8) + tile / 8;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;

    const int lane = (int)threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int p = wv >> 1, wave = wv & 1;  // K range, column half
    const int tid = (int)threadIdx.x & 127;  // thread within the range's pair of waves
    const int r16 = lane & 15, g = lane >> 4;
    uint8_t *const lds = lds_all + p * 2 * kBuf;
    const int kbs = p * L * SB;                                        // first block of the range
    const int ns = nst - p * L < L ? (nst - p * L > 0 ? nst - p * L : 0) : L;  // stages of the range

    // X: thread t stages 16-byte chunk t % 8 of tile row t / 8; W: chunks t + 128 j.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xq, (uint64_t)M * (uint64_t)K);
    const int xrow = tid >> 3, xc = tid & 7;
    const uint32_t xoff = m0 + xrow < M ? (uint32_t)(m0 + xrow) * (uint32_t)K + (uint32_t)xc * 16u : kOob;
    const int xlds = xrow * 128 + ((xc ^ ((xrow >> 1) & 7)) << 4);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w.qs, (uint64_t)N * (uint64_t)K);
    uint32_t woff[2];
    int wlds[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int q = tid + 128 * j, row = q >> 3, c = q & 7;
        woff[j] = n0 + row < N ? (uint32_t)(n0 + row) * (uint32_t)K + (uint32_t)c * 16u : kOob;
        wlds[j] = kXS + row * 128 + ((c ^ ((row >> 1) & 7)) << 4);
    }
    // Scales: thread t < 16 loads sx of tile row t (four blocks); thread 16 + u (u < 16)
    // loads dw of block u / 4 of the stage, columns 8 (u % 4) .. + 7, from the block-major
    // copy (the block index is a per-lane offset).
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(xs, (uint64_t)M * (uint64_t)nblk * 4u);
    const __amdgpu_buffer_rsrc_t dr = make_rsrc(w.d, (uint64_t)N * (uint64_t)nblk * 2u);
    const bool sthr = tid < 16, dthr = tid >= 16 && tid < 32;
    const int du = tid - 16, dcol = 8 * (du & 3), dblk = du >> 2;
    const uint32_t soff = sthr && m0 + tid < M ? (uint32_t)(m0 + tid) * (uint32_t)nblk * 4u : kOob;
    const uint32_t doff = dthr && n0 + dcol < N ? ((uint32_t)dblk * (uint32_t)N + (uint32_t)(n0 + dcol)) * 2u : kOob;

    struct Set {
        u32x4 x, w[2], s, d;
    };
    Set set[R];
    // Fixed per-lane offsets and the stage as the scalar offset, so the loads carry no
    // per-stage condition (a condition there became a branch, and the wait counts the
    // compiler derives across it waited for the first load of the same stage): stages past
    // the range take 2^30 (every offset then past the end of its buffer or inside it); bytes
    // past K in the last stage are never read by an MFMA.
    auto load = [&](int i, Set &S_) {
        const bool live = i < ns;
        const int kb0 = kbs + i * SB;
        const uint32_t kx = live ? (uint32_t)kb0 * 32u : 0x40000000u;
        S_.x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff, kx, 0));
#pragma unroll
        for (int j = 0; j < 2; j++)
            S_.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, woff[j], kx, 0));
        S_.s = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, soff, live ? (uint32_t)kb0 * 4u : 0x40000000u, 0));
        S_.d = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(dr, doff, live ? (uint32_t)kb0 * (uint32_t)N * 2u : 0x40000000u, 0));
    };
    auto store = [&](const Set &S_, int buf) {
        uint8_t *const b = lds + buf * kBuf;
        *reinterpret_cast<u32x4 *>(&b[xlds]) = S_.x;
#pragma unroll
        for (int j = 0; j < 2; j++) *reinterpret_cast<u32x4 *>(&b[wlds[j]]) = S_.w[j];
        if (sthr) {
            float *sx = reinterpret_cast<float *>(b + kXS + kWS) + tid;
            const f32x4 v = __builtin_bit_cast(f32x4, S_.s);
            sx[0 * BM] = v.x;
            sx[1 * BM] = v.y;
            sx[2 * BM] = v.z;
            sx[3 * BM] = v.w;
        } else if (dthr) {
            float *dw = reinterpret_cast<float *>(b + kXS + kWS + kSxS) + dblk * BN + dcol;
            // whole-vector casts only: this compiler's __builtin_bit_cast of one element of an
            // ext_vector lvalue (v.y, v[i]) reads element 0
            const f32x8 f = __builtin_convertvector(__builtin_bit_cast(f16x8, S_.d), f32x8);
            *reinterpret_cast<f32x4 *>(dw) = __builtin_shufflevector(f, f, 0, 1, 2, 3);
            *reinterpret_cast<f32x4 *>(dw + 4) = __builtin_shufflevector(f, f, 4, 5, 6, 7);
        }
    };
    // Operand lane (r, g): 8 bytes at k = 8 g of the block, i.e. half g % 2 of 16-byte chunk
    // 2 kb + g / 2 of the row.
    const int rb = 16 * wave + r16;
    const int asw = (r16 >> 1) & 7, bsw = (rb >> 1) & 7;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    auto mfma = [&](const uint8_t *b, int kb) {
        const int c = 2 * kb + (g >> 1), half = 8 * (g & 1);
        const long a = *reinterpret_cast<const long *>(&b[r16 * 128 + ((c ^ asw) << 4) + half]);
        const long q = *reinterpret_cast<const long *>(&b[kXS + rb * 128 + ((c ^ bsw) << 4) + half]);
        return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, q, i32x4s{0, 0, 0, 0}, 0, 0, 0);
    };
    // Scale products of the stage's four blocks on the matrix core: lane (g, r16) supplies sx
    // of tile row r16 and dw of column rb for block g, and v_mfma_f32_16x16x1_4b_f32 returns
    // the four 16 x 16 outer products (block kb in elements 4 kb .. 4 kb + 3) in the layout
    // of the int8 product, each element the fp32 product fl(sx * dw) (a0 * b0 + 0 rounded
    // once; the sign of a zero product is lost, which the fold cannot see).
    auto scales = [&](const uint8_t *b) {
        const float sx = reinterpret_cast<const float *>(b + kXS + kWS)[g * BM + r16];
        const float dw = reinterpret_cast<const float *>(b + kXS + kWS + kSxS)[g * BN + rb];
        return __builtin_amdgcn_mfma_f32_16x16x1f32(sx, dw, f32x16{}, 0, 0, 0);
    };
    // result element j: row 4 g + j, column lane % 16 of the wave's columns
    auto fold = [&](const i32x4s &I, const f32x16 &P, int kb) {
#pragma unroll
        for (int j = 0; j < 4; j++) acc[j] = __builtin_fmaf((float)I[j], P[4 * kb + j], acc[j]);
    };

#pragma unroll
    for (int r = 0; r < R; r++) {
        load(r, set[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
    store(set[0], 0);
    // Iteration i: the barrier publishes stage i (stored during iteration i - 1) and frees
    // the other buffer; the loads of stage i + R go into the set stage i came from; stage
    // i + 1 is stored while stage i is computed.
    for (int i0 = 0; i0 < L; i0 += R) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int i = i0 + r;  // i0 is a multiple of the even R: buffer i % 2 == r % 2
            __syncthreads();
            load(i + R, set[r]);
            __builtin_amdgcn_sched_barrier(0);
            store(set[(r + 1) % R], (r + 1) & 1);
            const uint8_t *b = lds + (r & 1) * kBuf;
            const int kb0 = kbs + i * SB;
            if (i >= ns) {
                // past the range: nothing to fold
            } else if (kb0 + SB <= nblk) {
                i32x4s I[SB];
#pragma unroll
                for (int kb = 0; kb < SB; kb++) I[kb] = mfma(b, kb);
                const f32x16 P = scales(b);
#pragma unroll
                for (int kb = 0; kb < SB; kb++) fold(I[kb], P, kb);
            } else {
                const f32x16 P = scales(b);
#pragma unroll
                for (int kb = 0; kb < SB; kb++)
                    if (kb0 + kb < nblk) fold(mfma(b, kb), P, kb);
            }
        }
    }
    const int col = n0 + rb;
    if constexpr (RG == 1) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = m0 + 4 * g + j;
            if (row < M && col < N) y[(int64_t)row * N + col] = acc[j];
        }
        return;
    }
    // ---- the partials of ranges 1, 2, 3 go through LDS; range 0 adds them in order
    __syncthreads();
    f32x4 *red = reinterpret_cast<f32x4 *>(lds_all);
    if (p > 0) red[((p - 1) * 2 + wave) * 64 + lane] = f32x4{acc[0], acc[1], acc[2], acc[3]};
    __syncthreads();
    if (p > 0) return;
    const f32x4 p1 = red[wave * 64 + lane], p2 = red[(2 + wave) * 64 + lane], p3 = red[(4 + wave) * 64 + lane];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int row = m0 + 4 * g + j;
        if (row < M && col < N) y[(int64_t)row * N + col] = ((acc[j] + p1[j]) + p2[j]) + p3[j];
    }
}

}  // namespace gw
}  // namespace j4q

namespace j4q {
namespace gw {

// Prefill GEMM, int8 variant above M = 256, with the tiles loaded straight into LDS and the
// fold of each block pair overlapped with the next pair's products (every output folded
// by one lane over all of K in block order: bit-identical to the oracle's emulation).
//  - Tile 64 x 128 per workgroup of 8 waves (two per SIMD); wave w owns the 32 x 32 outputs
//    of rows 32 (w % 2), columns 32 (w / 2). K advances in stages of four blocks (one 128-byte
//    line of every row).
//  - Every stage moves straight from global memory into one of three LDS stage buffers
//    (buffer_load ... lds, no VGPRs, no LDS stores): X as 64 rows and W as 128 rows of 128
//    bytes, 16-byte chunk c of row r at slot c ^ ((r / 2) % 8), so the 16 rows of one
//    quarter-wave of an operand read cover all 64 banks; then sx as [64 rows][4 blocks] fp32
//    and dw as [4 blocks][128 columns] fp16 (from the block-major copy). A lane loads the
//    global chunk that belongs at its LDS slot. Every wave issues four loads per stage (X, two
//    of W, a quarter of sx or of dw), so all waves wait for the same count and no load sits
//    behind a branch.
//  - Iteration i: wait for own stage-i loads, barrier, then stage i with the four loads of
//    stage i + 2 (into the buffers of stage i - 1; the ring's look-ahead past the end loads
//    the last stage again) between its steps. A stage reads a pair's operands a step before
//    its MFMAs and folds the pair before it in between, so the LDS latency, the matrix work
//    and the fold overlap in every wave (measured on MI355X at N = K = 4096, quantizer
//    included: M = 512 36.8 us and M = 2048 136 us, against 43.8 and 159 us for the same tile
//    loaded through registers and folded right after its own products; stages of eight blocks
//    with half the barriers ran 39.7 us at M = 512).
// Requires K % 32 == 0, N % 8 == 0, M * K < 2^31 and N * K < 2^31. Internal linkage: this header
// is included by more than one source.
[[maybe_unused]] static __global__ void __launch_bounds__(512)
gemm_i8_lds(QMat w, const int8_t *__restrict__ xq, const float *__restrict__ xsc, float *__restrict__ y, int M) {
    constexpr int BM = 64, BN = 128, SB = 4;  // rows, columns, blocks per stage
    constexpr int kX = BM * 128, kW = BN * 128, kSx = BM * SB * 4, kS = kSx + SB * BN * 2;
    __shared__ __attribute__((aligned(1024))) uint8_t xs0[kX], xs1[kX], xs2[kX];
    __shared__ __attribute__((aligned(1024))) uint8_t ws0[kW], ws1[kW], ws2[kW];
    __shared__ __attribute__((aligned(1024))) uint8_t ss0[kS], ss1[kS], ss2[kS];
    const int N = (int)w.rows, K = (int)w.cols, nblk = K / 32;
    const int nfull = nblk / SB, ns = (nblk + SB - 1) / SB;  // full stages, all stages
    const int mt = (M + BM - 1) / BM;
    // Workgroup b runs on XCD b % 8; each XCD takes a contiguous range of tiles (m fastest),
    // so the m tiles of the same W rows share an L2.
    const int total = (int)gridDim.x;
    int tile = (int)blockIdx.x;
    if (total % 8 == 0) tile = (tile % 8) * (total / 8) + tile / 8;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;

    const int lane = (int)threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wm = wave & 1, wn = wave >> 1, h = lane >> 5, l32 = lane & 31;

    // X: wave w fills rows 8 w .. 8 w + 7 (lane L the slot L % 8 of row 8 w + L / 8); W: load
    // j of wave w fills rows 8 (8 j + w) .. + 7.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xq, (uint64_t)M * (uint64_t)K);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w.qs, (uint64_t)N * (uint64_t)K);
    uint32_t xoff, woff[2];
    {
        const int row = 8 * wave + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
        xoff = m0 + row < M ? (uint32_t)(m0 + row) * (uint32_t)K + (uint32_t)c * 16u : kOob;
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = 8 * (8 * j + wave) + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
        woff[j] = n0 + row < N ? (uint32_t)(n0 + row) * (uint32_t)K + (uint32_t)c * 16u : kOob;
    }
    // Scales, 4 bytes per lane into 256-byte slot w of the stage's scale buffer:
    //  - waves 0..3: sx as [64 rows][4 blocks] fp32; wave q lane L: row 16 q + L / 4, block
    //    L % 4 of the stage;
    //  - waves 4..7: dw as [4 blocks][128 columns] fp16; wave 4 + q lane L: block q of the
    //    stage, columns 2 L and 2 L + 1 (N % 8 == 0 keeps the pair in range together).
    // Each wave picks its source (resource, lane offset, bytes per stage) once.
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(xsc, (uint64_t)M * (uint64_t)nblk * 4u);
    const __amdgpu_buffer_rsrc_t dr = make_rsrc(w.d, (uint64_t)N * (uint64_t)nblk * 2u);
    const bool sxw = wave < 4;
    const __amdgpu_buffer_rsrc_t cr = sxw ? sr : dr;
    uint32_t coff;
    {
        const int q = wave & 3, row = 16 * q + (lane >> 2), col = n0 + 2 * lane;
        coff = sxw ? (m0 + row < M ? (uint32_t)(m0 + row) * (uint32_t)nblk * 4u + (uint32_t)(lane & 3) * 4u : kOob)
                   : (col < N ? ((uint32_t)q * (uint32_t)N + (uint32_t)col) * 2u : kOob);
    }
    const uint32_t cstep = sxw ? 4u * SB : (uint32_t)N * 2u * SB;  // bytes per stage

    // Load j (0: X, 1 and 2: W, 3: scales) of stage i, clamped to the last stage (which the
    // ring's look-ahead past the end reads again: in range, never computed on).
    auto load = [&](int i, int j, uint8_t *xb, uint8_t *wb, uint8_t *sb) __attribute__((always_inline)) {
        const uint32_t st = (uint32_t)(i < ns ? i : ns - 1);
        if (j == 0) dma16(xr, xb + wave * 1024, xoff, st * 128u);
        else if (j == 1) dma16(wr, wb + wave * 1024, woff[0], st * 128u);
        else if (j == 2) dma16(wr, wb + (8 + wave) * 1024, woff[1], st * 128u);
        else dma4s(cr, sb + wave * 256, coff, st * cstep);
    };

    const int ra = 32 * wm + l32, rb = 32 * wn + l32;
    const int asw = (ra >> 1) & 7, bsw = (rb >> 1) & 7;
    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.f;
    // result element v: row 8 (v / 4) + 4 (lane / 32) + v % 4, column lane % 32
    auto fold = [&](const i32x16 &I, const f32x32 &Pr, int e) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[v] = __builtin_fmaf((float)I[v], Pr[16 * e + v], acc[v]);
    };
    struct Pair {
        i32x16 I0, I1;
        f32x32 Pr;
    };
    // operands of block pair p of a stage (blocks 2 p and 2 p + 1: chunks c0 and c1 of the
    // row's line)
    struct Ops {
        i32x4 a0, b0, a1, b1;
        float sx, dw;
    };
    auto read_ops = [&](const uint8_t *xb, const uint8_t *wb, const uint8_t *sb, int p, Ops &o) __attribute__((always_inline)) {
        const int c0 = 4 * p + h, c1 = 4 * p + 2 + h;
        o.a0 = *reinterpret_cast<const i32x4 *>(xb + ra * 128 + ((c0 ^ asw) << 4));
        o.b0 = *reinterpret_cast<const i32x4 *>(wb + rb * 128 + ((c0 ^ bsw) << 4));
        o.a1 = *reinterpret_cast<const i32x4 *>(xb + ra * 128 + ((c1 ^ asw) << 4));
        o.b1 = *reinterpret_cast<const i32x4 *>(wb + rb * 128 + ((c1 ^ bsw) << 4));
        o.sx = reinterpret_cast<const float *>(sb)[ra * SB + 2 * p + h];
        o.dw = half_bits_to_float(reinterpret_cast<const uint16_t *>(sb + kSx)[(2 * p + h) * BN + rb]);
    };
    // the pair's int8 products and scale products: lane (h, l32) supplies sx of row ra and
    // dw of column rb for block 2 p + h, and v_mfma_f32_32x32x1_2b_f32 returns both 32 x 32
    // outer products (block 2 p in elements 0..15, 2 p + 1 in 16..31) in the layout of the
    // int8 products
    auto products = [&](const Ops &o, Pair &out) __attribute__((always_inline)) {
        out.I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a0, o.b0, i32x16{}, 0, 0, 0);
        out.I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a1, o.b1, i32x16{}, 0, 0, 0);
        out.Pr = __builtin_amdgcn_mfma_f32_32x32x1f32(o.sx, o.dw, f32x32{}, 0, 0, 0);
    };
    // pa: pair 0 of the current stage; pb: the pair left for folding (pair 1 of the stage
    // before; zeros before the first stage, whose fold adds exact zeros: fma(0, 0, +0) = +0)
    Pair pa, pb;
    pb.I0 = i32x16{};
    pb.I1 = i32x16{};
    pb.Pr = f32x32{};
    // One stage, each step fenced from the next: read pair 0's operands, fold block 0 of the
    // left pair (its latency covers the reads), pair 0's products, read pair 1's operands,
    // fold block 1 of the left pair, pair 1's products, then fold pair 0 while pair 1's
    // products run; pair 1 is left for the next stage. The four loads of stage i + 2 sit
    // between the steps, so a wave never issues them back to back. (Every lambda here is
    // forced inline: the five calls of step were otherwise kept as calls, with a stack frame
    // in scratch memory.)
    auto stage = [&](const uint8_t *xb, const uint8_t *wb, const uint8_t *sb, int inext, uint8_t *xn, uint8_t *wn,
                     uint8_t *sn) __attribute__((always_inline)) {
        Ops o;
        wave_prio(3);
        read_ops(xb, wb, sb, 0, o);
        __builtin_amdgcn_sched_barrier(0);
        load(inext, 0, xn, wn, sn);
        __builtin_amdgcn_sched_barrier(0);
        fold(pb.I0, pb.Pr, 0);
        __builtin_amdgcn_sched_barrier(0);
        products(o, pa);
        __builtin_amdgcn_sched_barrier(0);
        wave_prio(2);
        read_ops(xb, wb, sb, 1, o);
        __builtin_amdgcn_sched_barrier(0);
        load(inext, 1, xn, wn, sn);
        __builtin_amdgcn_sched_barrier(0);
        fold(pb.I1, pb.Pr, 1);
        __builtin_amdgcn_sched_barrier(0);
        load(inext, 2, xn, wn, sn);
        __builtin_amdgcn_sched_barrier(0);
        products(o, pb);
        __builtin_amdgcn_sched_barrier(0);
        wave_prio(1);
        fold(pa.I0, pa.Pr, 0);
        __builtin_amdgcn_sched_barrier(0);
        wave_prio(0);
        load(inext, 3, xn, wn, sn);
        __builtin_amdgcn_sched_barrier(0);
        fold(pa.I1, pa.Pr, 1);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](int i, const uint8_t *xb, const uint8_t *wb, const uint8_t *sb, uint8_t *xn, uint8_t *wn,
                    uint8_t *sn) __attribute__((always_inline)) {
        wait_vm_lgkm0<4>();
        lds_barrier();
        stage(xb, wb, sb, i + 2, xn, wn, sn);
    };

#pragma unroll
    for (int j = 0; j < 4; j++) load(0, j, xs0, ws0, ss0);
#pragma unroll
    for (int j = 0; j < 4; j++) load(1, j, xs1, ws1, ss1);
    int i = 0;
    for (; i + 3 <= nfull; i += 3) {
        step(i, xs0, ws0, ss0, xs2, ws2, ss2);
        step(i + 1, xs1, ws1, ss1, xs0, ws0, ss0);
        step(i + 2, xs2, ws2, ss2, xs1, ws1, ss1);
    }
    if (i < nfull) {
        step(i, xs0, ws0, ss0, xs2, ws2, ss2);
        i++;
        if (i < nfull) {
            step(i, xs1, ws1, ss1, xs0, ws0, ss0);
            i++;
        }
    }
    fold(pb.I0, pb.Pr, 0);
    fold(pb.I1, pb.Pr, 1);
    // a last stage of 1..3 blocks (in buffer i % 3)
    if (nfull < ns) {
        const int r = i % 3;
        const uint8_t *xb = r == 0 ? xs0 : r == 1 ? xs1 : xs2;
        const uint8_t *wb = r == 0 ? ws0 : r == 1 ? ws1 : ws2;
        const uint8_t *sb = r == 0 ? ss0 : r == 1 ? ss1 : ss2;
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
        const int nb = nblk - nfull * SB;
        for (int p = 0; 2 * p < nb; p++) {
            Ops o;
            read_ops(xb, wb, sb, p, o);
            products(o, pa);
            fold(pa.I0, pa.Pr, 0);
            if (2 * p + 1 < nb) fold(pa.I1, pa.Pr, 1);
        }
    }
    const int col = n0 + rb;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int row = m0 + 32 * wm + 8 * (v >> 2) + 4 * h + (v & 3);
        if (row < M && col < N) y[(int64_t)row * N + col] = acc[v];
    }
}

}  // namespace gw
}  // namespace j4q

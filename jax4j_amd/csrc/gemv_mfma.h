// Batched decode GEMV on the matrix cores: y[b][n] = sum_k W[n, k] x[b][k] (+ add[b][n]) for
// a batch of B <= 16 activation rows, split-layout weights, with W streamed once for the batch.
//
// The vector-ALU GEMV (gemv_impl.h) streams W once per batch row: at B = 8 it reads every
// weight eight times. Here the products run on v_mfma_f32_16x16x32_f16 (16x16x16 for
// Q6_K's 16-element scale groups), the A operand carries all batch rows at once, and the
// VALU keeps only the unpack (5 bit operations per 8 Q4 weights) and one FMA per 32-block
// per C row.
//
// Exactness of the operands:
//  - Weights: a quant field AND-masked into the low bits of a 16-bit half is an fp16
//    subnormal q * 2^-24 (16 q * 2^-24 for a field at bits 4..7). MFMA consumes fp16
//    subnormals exactly, and products are exact in its fp32 accumulator.
//  - Activations: per batch row and wave, x is scaled by a power of two 2^e (max |x| * 2^e
//    over the wave's K slice in [2^14, 2^15), so nothing overflows fp16) and split into
//    x' = hi + lo, two fp16 values carrying 22 significant bits. For up to 8 batch rows the
//    A operand's 16 rows hold hi of batch rows 0..7 (rows 0..7) and lo (rows 8..15); rows
//    without a batch row are zero. For 16 batch rows there are two A operands (hi, lo) and
//    the lo MFMA takes the hi one's result as its C input. A wave's partial sums are
//    multiplied by 2^(24 - e) before the waves' sums are added, so each wave may pick its
//    own e.
//  - Offsets: the MFMA's C input carries -OFF * 2^-24 * sum(x') of the block, so the C
//    output is 2^-24 * sum (q - OFF) x' and one FMA with the block scale folds it into
//    the fp32 accumulator (Q4_K's min term is a second FMA).
//
// Work split: persistent workgroups take 16-row tiles; wave v of a workgroup owns a fixed K
// slice of IPW items (an item is 16 rows x 4 blocks; Q8_0: 2 blocks) for every tile, so it
// turns its slice of x into MFMA operands once. Lane l = 16 g + n loads 16 contiguous bytes
// of row n, unit g of the item; a 4 x 4 transpose across the 16-lane groups
// (v_permlane32_swap / v_permlane16_swap) leaves lane group g holding dword g of every
// unit, so each MFMA column sums one block of one row. The waves' partial sums of a tile are
// added through LDS in wave order, so results are deterministic. Two tiles' loads are in
// flight while a tile is computed.
#pragma once

#include "gemv_impl.h"

namespace j4q {
namespace gmf {

using gemv::f32x4;
using gemv::kOob;
using gemv::make_rsrc;
using gemv::Rsrc;
using gemv::u32x2;
using gemv::u32x4;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Weight loads keep the default cache policy, unlike the batch-1 kernel's non-temporal
// stream: a wave's item covers 64 bytes of each of 16 rows, half of a 128-byte line, and
// its next item the other half, which a non-temporal load fetched again (measured: B = 16
// decode step 2.64 -> 2.45 ms).
constexpr int kTile = 0;
// A load that is not `ok` takes the out-of-range lane offset (the scalar offset stays
// unconditional). The lane offset passes through an empty asm: with a select on the tile's
// liveness visible in the scalar offset, the compiler split some loads into two branches,
// and the wait counts it then derived waited for loads issued after the ones needed.
__device__ __forceinline__ uint32_t lane_off(uint32_t vo, bool ok) {
    uint32_t v = ok ? vo : kOob;
    asm("" : "+v"(v));
    return v;
}
__device__ __forceinline__ u32x4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, bool ok) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off(vo, ok), so, kTile));
}
__device__ __forceinline__ u32x2 ld64(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, bool ok) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, lane_off(vo, ok), so, kTile));
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, bool ok) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, lane_off(vo, ok), so, kTile);
}
__device__ __forceinline__ uint32_t ld16(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, bool ok) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, lane_off(vo, ok), so, kTile);
}

// On entry lane group g (lanes 16g..16g+15) holds v[0..3] = dwords 0..3 of its own unit g;
// on exit v[t] holds dword g of unit t.
__device__ __forceinline__ void xpose4(uint32_t (&v)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    v[0] = c[0];
    v[1] = c[1];
    v[2] = d[0];
    v[3] = d[1];
}

// o[t] = x of lane group t (same lane within the group), in every lane.
__device__ __forceinline__ void bcast4(float x, float (&o)[4]) {
    const uint32_t v = __builtin_bit_cast(uint32_t, x);
    const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // [g0 g1 g0 g1], [g2 g3 g2 g3]
    const auto b0 = __builtin_amdgcn_permlane16_swap(a[0], a[0], false, false);
    const auto b1 = __builtin_amdgcn_permlane16_swap(a[1], a[1], false, false);
    o[0] = __builtin_bit_cast(float, (uint32_t)b0[0]);
    o[1] = __builtin_bit_cast(float, (uint32_t)b0[1]);
    o[2] = __builtin_bit_cast(float, (uint32_t)b1[0]);
    o[3] = __builtin_bit_cast(float, (uint32_t)b1[1]);
}

// Q4 dword of lane group g: bytes 4g..4g+3 of a 16-byte chunk (byte i: lo nibble element
// i, hi nibble element 16 + i). Slots 0..7 of the B operand hold elements
// 4g + {0, 2, 1, 3, 16, 18, 17, 19}; slots 4..7 carry a factor 16.
__device__ __forceinline__ u32x4 q4_slots(uint32_t v) {
    const uint32_t t = v >> 8;
    return u32x4{v & 0x000F000Fu, t & 0x000F000Fu, v & 0x00F000F0u, t & 0x00F000F0u};
}

template <int FMT>
struct Fmt;

// Geometry shared by the formats: S blocks (32-element units) per item, the x scale of
// slots 4..7 (Q4-style fields sit at bits 4..7), and the per-block offset of the quants.
template <>
struct Fmt<Q4_0> {
    static constexpr int S = 4, GROUPS = 1;
    static constexpr float SIGMA = 0.0625f, OFF = 8.0f;
    u32x4 q;
    u32x2 d;  // unused: the tile's scales are loaded once per tile (see load_tile)
    __device__ __forceinline__ void load(const Rsrc &r, uint32_t row, uint32_t K, uint32_t g, int blk0, bool live) {
        q = ld128(r.qs, row * (K / 2u) + 16u * g, (uint32_t)blk0 * 16u, live);
    }
};

template <>
struct Fmt<Q4_K> {
    static constexpr int S = 4, GROUPS = 1;
    static constexpr float SIGMA = 0.0625f, OFF = 0.0f;
    u32x4 q;
    // superblock header d | dmin | D0 | D1 | D2 (split layout, j4q_common.h): loaded once per
    // tile, into item 0 (see load_tile)
    u32x4 meta;
    __device__ __forceinline__ void load(const Rsrc &r, uint32_t row, uint32_t K, uint32_t g, int blk0, bool live) {
        q = ld128(r.qs, row * (K / 2u) + 16u * g, (uint32_t)blk0 * 16u, live);
    }
};

template <>
struct Fmt<Q8_0> {
    static constexpr int S = 2, GROUPS = 1;
    static constexpr float SIGMA = 1.0f, OFF = 128.0f;
    u32x4 q;
    uint32_t d;  // fp16 d of blocks 0..1
    __device__ __forceinline__ void load(const Rsrc &r, uint32_t row, uint32_t K, uint32_t g, int blk0, bool live) {
        q = ld128(r.qs, row * K + 16u * g, (uint32_t)blk0 * 32u, live);
        d = ld32(r.sc, row * (K / 16u), (uint32_t)blk0 * 2u, live);
    }
};

template <>
struct Fmt<Q6_K> {
    static constexpr int S = 4, GROUPS = 2;
    static constexpr float SIGMA = 0.0625f, OFF = 32.0f;
    u32x4 q;
    u32x2 h;  // qh of chunk g (two dwords)
    // per tile, in item 0 (see load_tile): the int8 group scales of the wave's 16 blocks
    // (32 bytes) and the fp16 d of its two superblocks
    u32x4 sca, scb;
    uint32_t dd;
    __device__ __forceinline__ void load(const Rsrc &r, uint32_t row, uint32_t K, uint32_t g, int blk0, bool live) {
        q = ld128(r.qs, row * (K / 2u) + 16u * g, (uint32_t)blk0 * 16u, live);
        h = ld64(r.qh, row * (K / 4u) + 8u * g, (uint32_t)blk0 * 8u, live);
    }
};

// LDS plan for BB batch rows, WAVES waves of NBW blocks each, rounds of RT tiles (byte
// offsets):
//   xa   [WAVES * NBW][4 lane groups][2 BB rows][16 B]   hi/lo fp16 x image (a lane group's
//        16 lanes read 16 consecutive 16-byte rows: no LDS bank conflicts)
//   zero 512 BB bytes of zeros (A rows with no batch row read here, stride 0; none at
//        BB = 16, where every row carries one)
//   cin  [WAVES * NBW][G][BB] f32                         MFMA C input per block
//   part [RT][WAVES][BB][16] f32                          per-wave partial sums of a round
//   pa   [RT][BB * 16] f32x2                              prev / add of a round's outputs
template <int BB, int G, int WAVES, int NBW, int RT>
struct Plan {
    static constexpr int kXa = 0;
    static constexpr int kZero = kXa + WAVES * NBW * 128 * BB;
    static constexpr int kCin = kZero + (BB <= 8 ? 512 * BB : 0);
    static constexpr int kPart = kCin + WAVES * NBW * G * BB * 4;
    static constexpr int kPa = kPart + RT * WAVES * BB * 16 * 4;
    static constexpr int kBytes = kPa + RT * BB * 16 * 8;
};

// Tiles per round (one pair of barriers per round): 4, or 2 at BB = 16 or 16 waves (LDS).
template <int BB, int WAVES>
constexpr int round_tiles() { return BB <= 8 && WAVES <= 8 ? 4 : 2; }

// grid: (G_wg, R) persistent workgroups of WAVES waves; workgroup (w, r) takes 16-row tiles
// w, w + G_wg, ... of window r, the blocks [kb0 + r per, min(kb0 + (r + 1) per, nbe)) of
// every row. With part == nullptr (R = 1) the launch writes y = (W[:, window] x[window] +
// prev) + add, so windows can also run one launch after another, chained through prev
// (each adding the previous window's y, read before that element is rewritten) with the
// caller's add joining only in the last. With wsum, every window writes its own sums to
// wsum[r][b][row] (no prev, no add) and sum_windows_kernel adds them in window order.
// Wave v owns window blocks [v NBW, (v + 1) NBW) (NBW = IPW * S); blocks past the window
// load nothing and their x image is zero. Requires kb0 and kbn multiples of S (Q4_K, Q6_K:
// of 8, so every slice starts on a superblock), kbn <= WAVES * NBW and B <= BB. XREG keeps
// the wave's A operands and C inputs in registers for the whole kernel instead of
// re-reading them from LDS per tile.
// Wave priority p (0..3; s_setprio takes an immediate, so p must fold to a constant).
__device__ __forceinline__ void set_prio(int p) {
    if (p >= 3) __builtin_amdgcn_s_setprio(3);
    else if (p == 2) __builtin_amdgcn_s_setprio(2);
    else if (p == 1) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}

template <int FMT, int BB, int WAVES, int IPW, bool XREG, int TS, bool NB = false>
__global__ void __launch_bounds__(WAVES * 64)
gemv_mfma_kernel(QMat m, const float *__restrict__ x, const float *prev, const float *__restrict__ add, float *y,
                 int B, int kb0, int per, int nbe, float *__restrict__ wsum) {
    kb0 += (int)blockIdx.y * per;
    const int kbn = nbe - kb0 < per ? nbe - kb0 : per;
    if (wsum) {
        wsum += (int64_t)blockIdx.y * B * m.rows;
        prev = nullptr;
        add = nullptr;
    }
    using F = Fmt<FMT>;
    constexpr int S = F::S, G = F::GROUPS, NBW = IPW * S;
    constexpr bool W16 = BB == 16;  // two A operands (hi, lo) of 16 batch rows each
    static_assert(BB <= 8 || (W16 && !XREG), "BB up to 8, or 16 without XREG");
    constexpr int RT = round_tiles<BB, WAVES>();
    // the tile ring (TS tiles in flight) and the rounds (RT tiles per reduction) advance
    // together through super-rounds of SR tiles, so every ring slot index is a constant
    constexpr int SR = RT > TS ? RT : TS;
    static_assert(SR % RT == 0 && SR % TS == 0, "rounds and ring turns tile a super-round");
    using P = Plan<BB, G, WAVES, NBW, RT>;
    // threads (b, nn) < 16 BB fetch a tile's prev / add values with its weights
    static_assert(WAVES * 64 >= BB * 16, "one thread per output of a tile");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int K = (int)m.cols, N = (int)m.rows;
    const int tiles = (N + 15) / 16, nb = kb0 + kbn;  // blocks [kb0, nb) of every row
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int lw = wave * NBW;     // this wave's K slice: window blocks [lw, lw + NBW)
    const int blkw = kb0 + lw;     // ... and its first block in the row
    const Rsrc rs = gemv::rsrc_of(m, FMT);

    // ---- 1. x loads, then the first tiles' weight loads, then the x image ----------------
    // Each wave turns its own slice of x into MFMA operands, with its own power-of-two scale
    // per batch row (applied again when its partial sums are written), and needs no barrier.
    // The x loads go out first and the first TS tiles' weight loads right behind them, so
    // the weight stream starts while the image is built (the image waits only for x: loads
    // complete in issue order for the counter).
    constexpr int UNITS = BB * 4;                 // (batch row, lane group) units per block
    static_assert(64 % UNITS == 0, "a lane's units share one batch row");
    constexpr int XPL = (NBW * UNITS + 63) / 64;  // units per lane
    const int xb = (lane % UNITS) >> 2, xg = lane & 3;  // the batch row and lane group of this lane's units
    f32x4 xv[XPL][2];
    {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint64_t)B * (uint64_t)K * 4u);
#pragma unroll
        for (int i = 0; i < XPL; i++) {
            const int bl = (lane + 64 * i) / UNITS;
            const bool ok = lane + 64 * i < NBW * UNITS && xb < B && blkw + bl < nb;
            const uint32_t off = (uint32_t)(xb * K + (blkw + bl) * 32 + 4 * xg) * 4u;
            xv[i][0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? off : kOob, 0, 0));
            xv[i][1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? off + 64u : kOob, 0, 0));
        }
    }
    // Weight loads of the first TS tiles. The reducing threads (b, nn) = (tid / 16, tid % 16),
    // tid < 16 BB, also fetch prev[b][row] and add[b][row] with the tile's weights, so waiting
    // for them never drains the loads issued later.
    const __amdgpu_buffer_rsrc_t addr = make_rsrc(add ? (const void *)add : (const void *)y, add ? (uint64_t)B * N * 4u : 0);
    const __amdgpu_buffer_rsrc_t prevr = make_rsrc(prev ? (const void *)prev : (const void *)y, prev ? (uint64_t)B * N * 4u : 0);
    const int rb = (int)threadIdx.x >> 4, rn = (int)threadIdx.x & 15;
    // Q4_0 scales: one load per tile, lane group g fetching item g's four (16 rows x 32 B
    // instead of 16 rows x 8 B per item); process() broadcasts them across the groups.
    static_assert(FMT != Q4_0 || IPW <= 4, "Q4_0 tile scales cover four items");
    static_assert((FMT != Q4_K && FMT != Q6_K) || IPW * F::S == 16 || IPW * F::S == 8,
                  "Q4_K, Q6_K: a wave's slice is one or two superblocks");
    auto load_tile = [&](F (&it)[IPW], f32x2 &av, int tile) {
        const bool live = tile < tiles;
        const int r = tile * 16 + n;
        const uint32_t row = (uint32_t)(r < N ? r : N - 1);
#pragma unroll
        for (int i = 0; i < IPW; i++)
            it[i].load(rs, row, (uint32_t)K, (uint32_t)g, blkw + i * S, live && blkw + i * S < nb);
        if constexpr (FMT == Q4_0) {
            const bool ok = live && g < IPW && blkw + g * S < nb;
            it[0].d = ld64(rs.sc, row * (uint32_t)(K / 16) + 8u * (uint32_t)g, (uint32_t)blkw * 2u, ok);
        }
        // Q6_K: every lane fetches its row's scales of the slice (two 16-byte loads) and both
        // superblock scales: four loads per tile instead of two per item
        if constexpr (FMT == Q6_K) {
            const uint32_t so = (uint32_t)blkw * 2u;
            it[0].sca = ld128(rs.sc, row * (uint32_t)(K / 16), so, live);
            it[0].scb = ld128(rs.sc, row * (uint32_t)(K / 16) + 16u, so, live);
            // two 16-bit loads: a row's d section (K / 128 bytes) is only 2-byte aligned
            const uint32_t so_d = (uint32_t)(blkw >> 3) * 2u;
            it[0].dd = ld16(rs.d, row * (uint32_t)(K / 128), so_d, live) |
                       (ld16(rs.d, row * (uint32_t)(K / 128) + 2u, so_d, live) << 16);
        }
        // Q4_K: a slice of two superblocks: lane groups 0, 1 fetch the header of the first,
        // 2, 3 that of the second (16 rows x 32 contiguous bytes in one load); a slice of one
        // (16 rows): every lane fetches it, and no swap is needed
        if constexpr (FMT == Q4_K) {
            const uint32_t hs = NBW == 8 ? 0u : (uint32_t)g >> 1;
            const bool ok = live && blkw + 8 * (int)hs < nb;
            it[0].meta = ld128(rs.sc, row * (uint32_t)(K / 16) + 16u * hs, (uint32_t)(blkw >> 3) * 16u, ok);
        }
        const int ar = tile * 16 + rn;
        const bool aok = live && (int)threadIdx.x < 16 * BB && rb < B && ar < N;
        const uint32_t ao = aok ? (uint32_t)(rb * N + ar) * 4u : kOob;
        av.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prevr, ao, 0, 0));
        av.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(addr, ao, 0, 0));
    };
    F tset[TS][IPW];
    f32x2 avs[TS];
    const int t0 = (int)blockIdx.x, tstep = (int)gridDim.x;
    __builtin_amdgcn_sched_barrier(0);
    // In the loop without skip paths, one tile's loads after the other, as in the loop: with
    // the tiles' loads interleaved here, the wait counts the compiler derives for the loop
    // from both paths into it waited for the loads of the tile after the one needed (decode
    // steps B = 4 and 8 0.5-0.7 % faster). With skip paths those waits are set by the joins
    // instead, and the order cost a workgroup with a single tile (Q8_0 4096 x 4096 at B = 4
    // 9.7 -> 10.8 us).
#pragma unroll
    for (int k = 0; k < TS; k++) {
        load_tile(tset[k], avs[k], t0 + k * tstep);
        if constexpr (NB) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!NB) __builtin_amdgcn_sched_barrier(0);
    // zero block for the A rows and C inputs that carry no batch row (every wave writes the
    // same zeros, so no wave depends on another)
    if constexpr (!W16)
        for (int i = lane; i < 128 * BB; i += 64) reinterpret_cast<uint32_t *>(lds + P::kZero)[i] = 0u;
    // 2^e brings the maximum of |x| over the slice and the batch row into [2^14, 2^15): no
    // fp16 overflow, full precision. The lanes of a batch row are its quad and the lanes
    // 16, 32 or 48 further on (UNITS apart).
    int ex;
    float sx;
    {
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < XPL; i++) {
            const f32x4 a = xv[i][0], c = xv[i][1];
            v = fmaxf(v, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                               fmaxf(fmaxf(fabsf(c.x), fabsf(c.y)), fmaxf(fabsf(c.z), fabsf(c.w)))));
        }
        v = fmaxf(v, gemv::dpp<0xB1>(v));
        v = fmaxf(v, gemv::dpp<0x4E>(v));
        if constexpr (UNITS <= 32) {
            const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v), false, false);
            v = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
        }
        if constexpr (UNITS <= 16) {
            const auto sw = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v), false, false);
            v = fmaxf(__builtin_bit_cast(float, (uint32_t)sw[0]), __builtin_bit_cast(float, (uint32_t)sw[1]));
        }
        int e = 0;
        if (v > 0.f && v <= 3.402823466e38f) {
            int E;
            (void)frexpf(v, &E);
            e = 15 - E;
            e = e < -126 ? -126 : (e > 127 ? 127 : e);
        }
        ex = e;
        sx = ldexpf(1.0f, e);
    }
    {
        uint8_t *xa = lds + P::kXa;
        float *cin = reinterpret_cast<float *>(lds + P::kCin);
#pragma unroll
        for (int i = 0; i < XPL; i++) {
            const int u = lane + 64 * i;
            const int bl = u / UNITS, b = xb, gg = xg;
            const int blk = lw + bl;  // x image index (window-relative)
            const f32x4 a = xv[i][0] * sx, c = xv[i][1] * sx;
            const f32x4 hi4 = c * F::SIGMA;
            // slots: 4g + {0, 2, 1, 3}, then 16 + 4g + {0, 2, 1, 3} times SIGMA
            const float v[8] = {a.x, a.z, a.y, a.w, hi4.x, hi4.z, hi4.y, hi4.w};
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const h2 h = __builtin_convertvector((f32x2{v[2 * p], v[2 * p + 1]}), h2);
                const float r0 = v[2 * p] - (float)h.x, r1 = v[2 * p + 1] - (float)h.y;
                const h2 l = __builtin_convertvector((f32x2{r0, r1}), h2);
                hw[p] = __builtin_bit_cast(uint32_t, h);
                lw[p] = __builtin_bit_cast(uint32_t, l);
            }
            // block sums of x' over elements 0..15 and 16..31 (this unit's 4 + 4, then the quad)
            float s0 = (a.x + a.y) + (a.z + a.w), s1 = (c.x + c.y) + (c.z + c.w);
            s0 += gemv::dpp<0xB1>(s0);
            s0 += gemv::dpp<0x4E>(s0);
            s1 += gemv::dpp<0xB1>(s1);
            s1 += gemv::dpp<0x4E>(s1);
            if (u < NBW * UNITS) {
                *reinterpret_cast<u32x4 *>(xa + ((blk * 4 + gg) * 2 * BB + b) * 16) = u32x4{hw[0], hw[1], hw[2], hw[3]};
                *reinterpret_cast<u32x4 *>(xa + ((blk * 4 + gg) * 2 * BB + BB + b) * 16) = u32x4{lw[0], lw[1], lw[2], lw[3]};
                if (gg == 0) {
                    constexpr float U = 5.9604644775390625e-8f;  // 2^-24
                    if constexpr (G == 2) {
                        cin[(blk * 2 + 0) * BB + b] = -F::OFF * U * s0;
                        cin[(blk * 2 + 1) * BB + b] = -F::OFF * U * s1;
                    } else if constexpr (FMT == Q4_K) {
                        cin[blk * BB + b] = U * (s0 + s1);
                    } else {
                        cin[blk * BB + b] = -F::OFF * U * (s0 + s1);
                    }
                }
            }
        }
    }
    // The slice was written by this wave only; LDS operations of one wave complete in order,
    // so waiting for them is all the ordering the reads below need.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)

    // Lane (m, g) of the A operand: rows m < BB are hi of batch row m, rows 8..8+BB-1 lo of
    // batch row m - 8, other rows read the zero block with stride 0. The C rows of lane
    // group g are 4g..4g+3: groups 0 and 1 hold the hi rows of batch rows 4 (g & 1) + j and
    // take the C inputs; groups 2 and 3 hold the lo rows and read zeros.
    // BB = 16: row m of the first A operand is hi of batch row m, of the second lo of batch
    // row m; the second MFMA takes the first one's result as its C input, so every C row
    // 4g + j is batch row 4g + j (hi + lo) and every lane group takes the C inputs.
    const int mrow = lane & 15;
    int abase, astride;
    if constexpr (W16) {
        abase = P::kXa + ((lw * 4 + g) * 2 * BB + mrow) * 16;
        astride = 128 * BB;
    } else if (mrow < BB) {
        abase = P::kXa + ((lw * 4 + g) * 2 * BB + mrow) * 16;
        astride = 128 * BB;
    } else if (mrow >= 8 && mrow < 8 + BB) {
        abase = P::kXa + ((lw * 4 + g) * 2 * BB + BB + mrow - 8) * 16;
        astride = 128 * BB;
    } else {
        abase = P::kZero + g * 16;
        astride = 0;
    }
    constexpr int JB = BB < 4 ? BB : 4;  // C rows per lane that carry a batch row
    const int hb = W16 ? 4 * g : 4 * (g & 1);  // first batch row of this lane's C rows
    const bool hi_lane = W16 || (g < 2 && hb < BB);
    const int cbase = hi_lane ? P::kCin + (lw * G * BB + hb) * 4 : P::kZero;
    const int cstride = hi_lane ? G * BB * 4 : 0;
    auto a_op = [&](int bl) { return *reinterpret_cast<const h8 *>(lds + abase + bl * astride); };
    // BB = 16: the lo operand, BB rows further on in the lane group's image
    auto a_lo = [&](int bl) { return *reinterpret_cast<const h8 *>(lds + abase + BB * 16 + bl * astride); };
    auto c_in = [&](int bl, int k) { return reinterpret_cast<const float *>(lds + cbase + bl * cstride)[k]; };
    // registers keep only this lane's C inputs: k = j (group 0) and k = BB + j (Q6_K group 1)
    h8 areg[XREG ? NBW : 1];
    float creg[XREG ? NBW : 1][G * JB];
    if constexpr (XREG) {
#pragma unroll
        for (int bl = 0; bl < NBW; bl++) {
            areg[bl] = a_op(bl);
#pragma unroll
            for (int kk = 0; kk < G * JB; kk++) creg[bl][kk] = c_in(bl, kk < JB ? kk : BB + kk - JB);
        }
    }

    // per-batch-row factor that undoes this wave's x scale (2^-e); the 2^24 of the weights is
    // applied as a separate exact product, since 2^(24 - e) overflows for a slice maximum
    // of 2^118 or more (e <= -104)
    // (batch row bb's exponent is that of lane 4 bb)
    float wscale[BB];
#pragma unroll
    for (int bb = 0; bb < BB; bb++) wscale[bb] = ldexpf(1.0f, -__builtin_amdgcn_readlane(ex, 4 * bb));

    auto A = [&](int bl) -> h8 {
        if constexpr (XREG) return areg[bl];
        else return a_op(bl);
    };
    auto C = [&](int bl, int k) -> float {
        if constexpr (XREG) return creg[bl][k < BB ? k : JB + k - BB];
        else return c_in(bl, k);
    };

    // ---- 3. per tile: transpose, unpack, MFMA, block scale; partials through LDS ----------
    float *part = reinterpret_cast<float *>(lds + P::kPart);
    f32x2 *pa = reinterpret_cast<f32x2 *>(lds + P::kPa);
    auto process = [&](const F (&it)[IPW], f32x2 av, int slot) {
        float acc[JB], corr[JB];
#pragma unroll
        for (int j = 0; j < JB; j++) acc[j] = corr[j] = 0.f;
        // Q4_K: the min terms sum_blocks dmin * m * sum(x') as a 16 x 16 x 4 fp32 MFMA per
        // item (A: block sums of the hi batch rows, B: dmin * m of each row's 4 blocks), in
        // the result layout of the block products
        f32x4 corr4 = {0.f, 0.f, 0.f, 0.f};
        // Q4_K: the slice's superblock headers in every lane: with two, one swap of the lane
        // halves per dword (hdr[0] from groups 0, 1; hdr[1] from groups 2, 3)
        uint32_t hdr[2][4] = {};
        if constexpr (FMT == Q4_K) {
            const uint32_t m4[4] = {it[0].meta.x, it[0].meta.y, it[0].meta.z, it[0].meta.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if constexpr (NBW == 8) {
                    hdr[0][k] = m4[k];
                } else {
                    const auto sw = __builtin_amdgcn_permlane32_swap(m4[k], m4[k], false, false);
                    hdr[0][k] = sw[0];
                    hdr[1][k] = sw[1];
                }
            }
        }
        // Q4_0: item i's scales live in lane group i of it[0].d; broadcast them to all groups
        uint32_t bd[4][2];
        if constexpr (FMT == Q4_0) {
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const uint32_t v = w ? it[0].d.y : it[0].d.x;
                const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // [g0 g1 g0 g1], [g2 g3 g2 g3]
                const auto b0 = __builtin_amdgcn_permlane16_swap(a[0], a[0], false, false);
                const auto b1 = __builtin_amdgcn_permlane16_swap(a[1], a[1], false, false);
                bd[0][w] = b0[0];
                bd[1][w] = b0[1];
                bd[2][w] = b1[0];
                bd[3][w] = b1[1];
            }
        }
#pragma unroll
        for (int i = 0; i < IPW; i++) {
            const int blk0 = blkw + i * S;
            if constexpr (FMT == Q4_0 || FMT == Q4_K) {
                uint32_t v[4] = {it[i].q.x, it[i].q.y, it[i].q.z, it[i].q.w};
                xpose4(v);
                // Q4_K: lane group g decodes the scale and min of block g of the item; the
                // scales go to every group, the mins feed the min-term MFMA in place
                float dsck[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (FMT == Q4_K) {
                    const uint32_t *mt = hdr[(i * S) >> 3];
                    const int sj = (blk0 & 7) + g;
                    const f32x2 dm2 = __builtin_convertvector(__builtin_bit_cast(h2, mt[0]), f32x2);
                    const uint32_t scj = __builtin_amdgcn_ubfe(mt[1], 4 * sj, 4) | (__builtin_amdgcn_ubfe(mt[3], 2 * sj, 2) << 4);
                    const uint32_t mnj = __builtin_amdgcn_ubfe(mt[2], 4 * sj, 4) | (__builtin_amdgcn_ubfe(mt[3], 16 + 2 * sj, 2) << 4);
                    bcast4(dm2.x * (float)scj, dsck);
                    const float sa = mrow < BB ? reinterpret_cast<const float *>(lds + P::kCin)[(lw + i * S + g) * BB + mrow] : 0.f;
                    corr4 = __builtin_amdgcn_mfma_f32_16x16x4f32(sa, dm2.y * (float)mnj, corr4, 0, 0, 0);
                }
                f32x4 c[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int bl = i * S + t;
                    c[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                    if constexpr (FMT == Q4_0) {
#pragma unroll
                        for (int j = 0; j < JB; j++) c[t][j] = C(bl, j);
                    }
                    const h8 bq = __builtin_bit_cast(h8, q4_slots(v[t]));
                    c[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A(bl), bq, c[t], 0, 0, 0);
                    if constexpr (W16) c[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo(bl), bq, c[t], 0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    if constexpr (FMT == Q4_0) {
                        const uint32_t dw = bd[i][t >> 1];
                        const float df = (float)__builtin_bit_cast(h2, dw)[t & 1];
#pragma unroll
                        for (int j = 0; j < JB; j++) acc[j] = __builtin_fmaf(df, c[t][j], acc[j]);
                    } else {
#pragma unroll
                        for (int j = 0; j < JB; j++) acc[j] = __builtin_fmaf(dsck[t], c[t][j], acc[j]);
                    }
                }
            } else if constexpr (FMT == Q8_0) {
                uint32_t v[4] = {it[i].q.x, it[i].q.y, it[i].q.z, it[i].q.w};
                xpose4(v);
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int bl = i * S + t;
                    const uint32_t ua = v[2 * t] ^ 0x80808080u, ub = v[2 * t + 1] ^ 0x80808080u;
                    const u32x4 sl = {ua & 0x00FF00FFu, (ua >> 8) & 0x00FF00FFu, ub & 0x00FF00FFu, (ub >> 8) & 0x00FF00FFu};
                    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < JB; j++) c[j] = C(bl, j);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A(bl), __builtin_bit_cast(h8, sl), c, 0, 0, 0);
                    if constexpr (W16) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo(bl), __builtin_bit_cast(h8, sl), c, 0, 0, 0);
                    const float df = (float)__builtin_bit_cast(h2, it[i].d)[t];
#pragma unroll
                    for (int j = 0; j < JB; j++) acc[j] = __builtin_fmaf(df, c[j], acc[j]);
                }
            } else {  // Q6_K
                uint32_t v[4] = {it[i].q.x, it[i].q.y, it[i].q.z, it[i].q.w};
                xpose4(v);
                // qh: lane group g holds dwords {0, 1} of chunk g; chunk t needs dword g >> 1
                // of chunk t, rotated right by 8 when g is odd.
                const auto hs = __builtin_amdgcn_permlane32_swap(it[i].h.x, it[i].h.y, false, false);
                const auto e0 = __builtin_amdgcn_permlane16_swap(hs[0], hs[0], false, false);
                const auto e1 = __builtin_amdgcn_permlane16_swap(hs[1], hs[1], false, false);
                const uint32_t hq[4] = {e0[0], e0[1], e1[0], e1[1]};
                const float df = (float)__builtin_bit_cast(_Float16, (uint16_t)(it[0].dd >> (16 * ((i * S) >> 3))));
                // scale dwords 2 i, 2 i + 1 of the slice's eight
                const uint32_t sc2[2] = {i < 2 ? it[0].sca[(2 * i) & 3] : it[0].scb[(2 * i) & 3],
                                         i < 2 ? it[0].sca[(2 * i + 1) & 3] : it[0].scb[(2 * i + 1) & 3]};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int bl = i * S + t;
                    const uint32_t q = v[t];
                    const uint32_t hw = __builtin_amdgcn_alignbit(hq[t], hq[t], (uint32_t)(g & 1) * 8u);
                    const uint32_t tq = q >> 8, hsh = hw >> 2;
                    const uint32_t p0 = (q & 0x000F000Fu) | (hw & 0x00300030u);
                    const uint32_t p1 = (q & 0x00F000F0u) | (hw & 0x03000300u);
                    const uint32_t p2 = (tq & 0x000F000Fu) | (hsh & 0x00300030u);
                    const uint32_t p3 = (tq & 0x00F000F0u) | (hsh & 0x03000300u);
                    const h8 aop = A(bl);
                    f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int j = 0; j < JB; j++) {
                        c0[j] = C(bl, j);
                        c1[j] = C(bl, BB + j);
                    }
                    const h4 b0 = __builtin_bit_cast(h4, u32x2{p0, p2}), b1 = __builtin_bit_cast(h4, u32x2{p1, p3});
                    c0 = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_shufflevector(aop, aop, 0, 1, 2, 3), b0, c0, 0, 0, 0);
                    c1 = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_shufflevector(aop, aop, 4, 5, 6, 7), b1, c1, 0, 0, 0);
                    if constexpr (W16) {
                        const h8 alo = a_lo(bl);
                        c0 = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_shufflevector(alo, alo, 0, 1, 2, 3), b0, c0, 0, 0, 0);
                        c1 = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_shufflevector(alo, alo, 4, 5, 6, 7), b1, c1, 0, 0, 0);
                    }
                    const uint32_t scw = sc2[t >> 1];
                    const float s0 = df * (float)(int8_t)(scw >> (16 * (t & 1))),
                                s1 = df * (float)(int8_t)(scw >> (16 * (t & 1) + 8));
#pragma unroll
                    for (int j = 0; j < JB; j++) acc[j] = __builtin_fmaf(s1, c1[j], __builtin_fmaf(s0, c0[j], acc[j]));
                }
            }
        }
        // hi + lo (BB <= 8: lanes 32..63 hold the lo rows of the batch rows in lanes 0..31)
        float *pp = part + slot * (WAVES * BB * 16);
#pragma unroll
        for (int j = 0; j < JB; j++) {
            float v = acc[j] - (FMT == Q4_K ? corr4[j] : corr[j]);
            if constexpr (!W16) {
                const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                                 __builtin_bit_cast(uint32_t, v), false, false);
                v += __builtin_bit_cast(float, (uint32_t)sw[1]);
            }
            float ws = 0.f;
#pragma unroll
            for (int bb = 0; bb < BB; bb++) ws = (bb == hb + j) ? wscale[bb] : ws;
            if (hi_lane) pp[(wave * BB + hb + j) * 16 + n] = (v * 16777216.0f) * ws;
        }
        // the tile's prev / add values, fetched with its weights by threads (b, nn)
        if ((int)threadIdx.x < BB * 16) pa[slot * BB * 16 + threadIdx.x] = av;
    };
    // End of a round of ns tiles starting at tile t: thread (k, b, nn) adds the waves'
    // partials of output (b, row 16 (t + k tstep) + nn) in wave order. The second barrier
    // keeps the slots until every reader is done.
    // The round's ns x BB x 16 outputs are dealt to the threads (more outputs than threads
    // when the workgroup is small: 4 waves at BB = 16 take one tile per pass).
    auto finish = [&](int t, int ns) {
        __syncthreads();
        for (int i = (int)threadIdx.x; i < ns * BB * 16; i += WAVES * 64) {
            const int k = i / (BB * 16), o = i % (BB * 16);
            const int b = o >> 4, nn = o & 15;
            const float *pp = part + k * (WAVES * BB * 16);
            float s = 0.f;
            for (int w = 0; w < WAVES; w++) s += pp[(w * BB + b) * 16 + nn];
            const f32x2 av = pa[k * BB * 16 + o];
            const int r = (t + k * tstep) * 16 + nn;
            // the previous window's sum first, then add on its own: fl(fl(W.x) + add)
            if (prev) s += av.x;
            if (b < B && r < N) {
                if (wsum) wsum[(int64_t)b * N + r] = s;
                else y[(int64_t)b * N + r] = add ? s + av.y : s;
            }
        }
        __syncthreads();
    };

    // TS register sets form a ring: the next TS - 1 tiles' loads are in flight while a tile is
    // computed. Waves run through a round of RT tiles without waiting for each other; the
    // partial sums meet at the round's end. The tile loop is workgroup-uniform, so every
    // wave reaches each barrier. A wave's priority falls with its place in the round (RT - 1
    // on the round's first tile, 0 on its last), so a wave that is behind issues before one
    // that is ahead and the waves of a SIMD reach the barrier together. Measured (A/B pairs on
    // one box, five rounds): decode step B = 4 1.819-1.852 -> 1.784-1.805 ms, B = 8
    // 2.063-2.070 -> 2.015-2.045 ms, B = 16 2.267-2.300 -> 2.254-2.267 ms.
    for (int t = t0; t < tiles; t += SR * tstep) {
#pragma unroll
        for (int rr = 0; rr < SR / RT; rr++) {
            const int tr = t + rr * RT * tstep;
            if (tr >= tiles) break;
            int ns = 0;
#pragma unroll
            for (int k = 0; k < RT; k++) {
                const int tk = tr + k * tstep;
                const int slot = (rr * RT + k) % TS;
                if constexpr (NB) {
                    // every slot's loads on every path (past the last tile they load
                    // nothing): a skip path joined into the following tiles' code makes the
                    // compiler's merged wait counts wait for the next tile's loads
                    if (tk < tiles) {
                        set_prio(RT - 1 - k);
                        process(tset[slot], avs[slot], k);
                        ns = k + 1;
                    }
                    load_tile(tset[slot], avs[slot], tk + TS * tstep);
                } else {
                    if (tk >= tiles) break;
                    set_prio(RT - 1 - k);
                    process(tset[slot], avs[slot], k);
                    load_tile(tset[slot], avs[slot], tk + TS * tstep);
                    ns = k + 1;
                }
            }
            finish(tr, ns);
        }
    }
}

// One launch: `windows` windows of `per` blocks from kb0 (the last ends at nbe), `grid`
// workgroups each; several windows need `part` (windows x B x rows floats).
template <int FMT, int BB, int WAVES, int IPW, bool XREG, int TS = 2, bool NB = false>
hipError_t launch_k(const QMat &m, const float *x, const float *add, float *y, int B, int grid, hipStream_t s, int kb0,
                    int per, int nbe, const float *prev, int windows, float *part) {
    constexpr int NBW = IPW * Fmt<FMT>::S;
    constexpr int lds = Plan<BB, Fmt<FMT>::GROUPS, WAVES, NBW, round_tiles<BB, WAVES>()>::kBytes;
    static_assert(lds <= 160 * 1024, "LDS of one workgroup");
    if (windows > 1 && !part) return hipErrorInvalidValue;
    gemv_mfma_kernel<FMT, BB, WAVES, IPW, XREG, TS, NB><<<dim3(grid, windows), WAVES * 64, lds, s>>>(
        m, x, prev, add, y, B, kb0, per, nbe, windows > 1 ? part : nullptr);
    return hipGetLastError();
}

// y[i] = ((part[0][i] + part[1][i]) + ...) + add[i] for i < n (= B x rows): the windows'
// sums in window order (the same additions as windows chained through prev), then the add
// on its own. Each element is read and written by one thread, so add may be y itself. A
// thread takes 4 consecutive elements (one element when n or an address does not allow
// float4 access) and issues the loads of up to 8 windows before it adds any of them, so the
// latencies overlap instead of adding up window by window.
__global__ void __launch_bounds__(256)
sum_windows_kernel(const float *__restrict__ part, int windows, int64_t n, const float *add, float *y) {
    // vector path for whole float4 rows at 16-byte aligned addresses
    const bool vec = (n & 3) == 0 && (((uintptr_t)part | (uintptr_t)add | (uintptr_t)y) & 15u) == 0;
    const int64_t n4 = vec ? n / 4 : 0;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        // add is fetched with the first windows (it is added last)
        const f32x4 a = add ? reinterpret_cast<const f32x4 *>(add)[i] : f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 v = reinterpret_cast<const f32x4 *>(part)[i];
        for (int r0 = 1; r0 < windows; r0 += 8) {
            f32x4 t[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (r0 + k < windows) t[k] = reinterpret_cast<const f32x4 *>(part + (int64_t)(r0 + k) * n)[i];
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (r0 + k < windows) v += t[k];
        }
        if (add) v += a;
        reinterpret_cast<f32x4 *>(y)[i] = v;
    }
    for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
        float v = part[i];
        for (int r = 1; r < windows; r++) v += part[(int64_t)r * n + i];
        if (add) v += add[i];
        y[i] = v;
    }
}

}  // namespace gmf
}  // namespace j4q

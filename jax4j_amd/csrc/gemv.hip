// Decode GEMV dispatch: picks the row-group size R, waves per workgroup and grid size of
// the persistent GEMV kernel (gemv_impl.h) for each format and shape.
#include <atomic>

#include "gemv_impl.h"
#include "gemv_mfma.h"
#include "jax4j_mi355x.h"

namespace j4q {
namespace gemv {
TraceSink g_gemv_trace = {nullptr, 0};
}  // namespace gemv

void gemv_set_trace(uint64_t *words, int64_t n) {
    gemv::g_gemv_trace.p = n >= 4 ? words : nullptr;
    gemv::g_gemv_trace.waves = n >= 4 ? (int)(n / 4 < 0x7fffffff ? n / 4 : 0x7fffffff) : 0;
}

int64_t gemv_get_trace(uint64_t **words) {
    *words = gemv::g_gemv_trace.p;
    return gemv::g_gemv_trace.p ? 4 * (int64_t)gemv::g_gemv_trace.waves : 0;
}

// Widest K one vector-ALU launch covers (x image in LDS); a wider K runs as column windows.
int64_t gemv_single_pass_cols() { return gemv::kMaxWindow; }

namespace {

// Launch shape, from measured sweeps on MI355X (one row per group, two register sets in
// flight, ~62 VGPRs per wave): for windows of K <= 4096, 8 waves per workgroup and 2
// workgroups per CU (the workgroups after the first on a CU stage x behind the weight
// stream of those before them: against 4 per CU, the decode step 1.256-1.259 -> 1.249-1.251
// ms by median over six A/B rounds on one box, Q4_K 14336 x 4096 9.2 -> 9.0 us; 1 or 3 per
// CU and one 16-wave workgroup per CU were slower), its waves taking row groups from the
// workgroup's pool (gemv_kernel DYN; against fixed shares, Q4_0 11008 x 4096 8.0 -> 7.6 us,
// Q8_0 4096 x 4096 6.4 -> 6.2 us, Q4_K 14336 x 4096 9.0 -> 8.75 us, decode step 1.21 -> 1.19
// ms; pooled 16-wave workgroups, one per CU, were slower), or for matrices of at least 16384 rows one
// workgroup of 16 waves per CU (every CU stages x once, at the start: with two workgroups
// per CU the second one's x loads queued behind the first one's weight stream; the
// Llama-3-8B decode step 1.226-1.232 -> 1.213-1.219 ms in an A/B on one box, the fused
// gate|up and the output head taking it), its waves taking row groups from the workgroup's
// pool (gemv_kernel DYN: the fused gate|up 14.9-15.0 -> 13.7 us, the step 1.21-1.23 ->
// 1.16-1.17 ms in an A/B on one box; 16 waves in two workgroups per CU had won
// 1.271 -> 1.260 ms over 8-wave workgroups; a ring of 3 or 4 register sets at one workgroup
// per CU lost, 1.25 and 1.28 ms; q|k|v at 16 waves lost, 6.3 -> 7.1 us); for K <= 8192, 2
// workgroups per CU; for larger windows (an x image of up to 139 KB), 16 waves in one
// workgroup per CU. The grid never exceeds what is resident at once, so x is staged once per
// workgroup.
template <int FMT>
hipError_t launch_window(const QMat &m, const float *x, const float *prev, const float *add, float *y, int batch,
                         int cus, int64_t c0, int64_t kw, hipStream_t s) {
    if (kw <= 4096)
        return m.rows >= 16384 ? gemv::launch<FMT, 1, 16, 2, true>(m, x, prev, add, y, batch, cus, c0, kw, s)
                               : gemv::launch<FMT, 1, 8, 2, true>(m, x, prev, add, y, batch, 2 * cus, c0, kw, s);
    if (kw <= 8192) return gemv::launch<FMT, 1, 8, 2>(m, x, prev, add, y, batch, 2 * cus, c0, kw, s);
    return gemv::launch<FMT, 1, 16, 2>(m, x, prev, add, y, batch, cus, c0, kw, s);
}

// K up to 32768 in one launch; wider K as equal windows of whole 2048-column steps, each
// adding the previous window's y (prev), the caller's add joining only in the last one.
// Callers keep an add that overlaps y to a single window (it would be read after y was
// rewritten).
template <int FMT>
hipError_t launch_fmt(const QMat &m, const float *x, const float *add, float *y, int batch, int cus, hipStream_t s) {
    const int64_t K = m.cols;
    if (K <= gemv::kMaxWindow) return launch_window<FMT>(m, x, nullptr, add, y, batch, cus, 0, K, s);
    const int64_t windows = (K + gemv::kMaxWindow - 1) / gemv::kMaxWindow;
    const int64_t per = ((K + windows - 1) / windows + 2047) / 2048 * 2048;
    for (int64_t c0 = 0; c0 < K; c0 += per) {
        const int64_t kw = K - c0 < per ? K - c0 : per;
        const bool last = c0 + kw >= K;
        const hipError_t e = launch_window<FMT>(m, x, c0 ? y : nullptr, last ? add : nullptr, y, batch, cus, c0, kw, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int g_cus = 256;

// Waves per workgroup and items per wave of launch_mfma (waves x items x blocks per item is
// the launch window):
//  - up to 8 rows: windows of 128 blocks (4096 columns); 16 waves for Q8_0 and Q4_0 (half
//    the items per wave, twice the waves to hide the load latency: Q8_0 4096 x 4096 at B = 8
//    12.8 -> 10.9 us, Q4_0 11008 x 4096 12.4 -> 12.0 us; Q4_K was 2 % slower and Q6_K spilled
//    registers), else 8;
//  - 9..16 rows: 8 waves of 8 blocks, windows of 64 blocks (2048 columns, a 128 KB x image
//    and ~152-156 KB of LDS in all, one workgroup per CU): half the windows of 4 waves over
//    1024 columns (two workgroups per CU), so half the partial sums for sum_windows_kernel
//    to add, with the same 8 waves per CU. Measured on the B = 16 decode step (A/B on one
//    box, all windows of a matrix in one launch): 2.29-2.31 ms against 2.43-2.46 ms for 4
//    waves (the two were level, 3.42 against 3.41 ms, before the tile loop's wait-count
//    fixes); 8 waves of 4 blocks over 1024-column windows (16 waves per CU) took 3.02 ms
//    against 2.69 ms for 4 waves of 8.
template <int FMT, int BB>
constexpr int mfma_waves() { return BB > 8 ? 8 : (FMT == Q8_0 || FMT == Q4_0) ? 16 : 8; }
template <int FMT, int BB>
constexpr int mfma_ipw() { return BB > 8 ? (FMT == Q8_0 ? 4 : 2) : (FMT == Q8_0 ? 8 : 4) * 8 / mfma_waves<FMT, BB>(); }
// Tiles in flight per wave: two (measured on the B = 16 decode step: 3.37 ms at 2, 3.52 ms
// at 4, 3.78 ms at 8).
template <int FMT, int BB>
constexpr int mfma_ring() { return 2; }
template <int FMT, int BB>
constexpr int mfma_window() { return mfma_waves<FMT, BB>() * mfma_ipw<FMT, BB>() * (FMT == Q8_0 ? 2 : 4); }

// Column windows of a matrix for a launch of BB batch rows: windows of at most CAP blocks,
// equal, aligned to whole items (K-quants: to whole 8-block superblocks, so each wave's
// slice starts a superblock).
template <int FMT, int BB>
void mfma_windows(const QMat &m, int &windows, int &per) {
    constexpr int S = FMT == Q8_0 ? 2 : 4, CAP = mfma_window<FMT, BB>();
    constexpr int AL = FMT == Q4_K || FMT == Q6_K ? 8 : S;
    static_assert(CAP % AL == 0, "windows fit the cap");
    const int nb = (int)(m.cols / 32);
    windows = (nb + CAP - 1) / CAP;
    per = ((nb + windows - 1) / windows + AL - 1) / AL * AL;
    windows = (nb + per - 1) / per;
}

// Workgroups of launch_mfma<FMT, BB>'s kernel that one CU holds at once, by LDS and by
// registers (hipOccupancyMaxActiveBlocksPerMultiprocessor at init); the LDS bound alone
// would launch two workgroups per CU where registers admit one (Q4_K with 8 waves of ~170
// VGPRs at 4 rows, Q4_0 with 16 waves of ~100), and the second half of the grid would run
// only after the first.
int g_mfma_resident[4][3];  // [Q4_0, Q8_0, Q4_K, Q6_K][BB 4, 8, 16]; 0 = not measured

constexpr int fmt_slot(int fmt) { return fmt == Q4_0 ? 0 : fmt == Q8_0 ? 1 : fmt == Q4_K ? 2 : 3; }
constexpr int bb_slot(int bb) { return bb <= 4 ? 0 : bb <= 8 ? 1 : 2; }

template <int FMT, int BB>
constexpr int mfma_lds() {
    return gmf::Plan<BB, gmf::Fmt<FMT>::GROUPS, mfma_waves<FMT, BB>(), mfma_ipw<FMT, BB>() * (FMT == Q8_0 ? 2 : 4),
                     gmf::round_tiles<BB, mfma_waves<FMT, BB>()>()>::kBytes;
}

template <int FMT, int BB>
void measure_resident() {
    constexpr int W = mfma_waves<FMT, BB>();
    int n = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &n, (const void *)gmf::gemv_mfma_kernel<FMT, BB, W, mfma_ipw<FMT, BB>(), false, mfma_ring<FMT, BB>()>, W * 64,
        mfma_lds<FMT, BB>());
    g_mfma_resident[fmt_slot(FMT)][bb_slot(BB)] = e == hipSuccess && n > 0 ? n : 0;
}

template <int FMT>
void measure_resident_fmt() {
    measure_resident<FMT, 4>();
    measure_resident<FMT, 8>();
    measure_resident<FMT, 16>();
}

// Batched GEMV on the matrix cores (gemv_mfma.h) for up to 16 batch rows per launch,
// persistent workgroups of 16-row tiles, each launch window of up to 128 blocks (4096
// columns; 64 at 16 rows) split into one slice per wave. A wider K has several windows:
// with a workspace they all run in one launch (grid.y = window, about CUs / windows
// workgroups each, every CU holding one window's x image) and sum_windows_kernel adds
// their sums in window order; without one they run as launches chained through prev (the
// same additions in the same order). Measured on MI355X (Q4_0 11008 x 4096): B = 4 10.8 us,
// B = 8 12.4 us, against 22 us and 41 us for one vector-ALU pass per batch row; at B <= 2
// the two are level.
template <int FMT, int BB>
hipError_t launch_mfma(const QMat &m, const float *x, const float *add, float *y, int b, const Workspace &ws,
                       hipStream_t s) {
    constexpr int W = mfma_waves<FMT, BB>(), IPW = mfma_ipw<FMT, BB>(), S = FMT == Q8_0 ? 2 : 4;
    constexpr int CAP = mfma_window<FMT, BB>();
    static_assert(CAP == W * IPW * S && CAP == (BB > 8 ? 8 * W : 128), "window = waves x items per wave x blocks per item");
    const int tiles = (int)((m.rows + 15) / 16);
    const int nb = (int)(m.cols / 32);
    int windows, per;
    mfma_windows<FMT, BB>(m, windows, per);
    const uint64_t need = windows > 1 ? (uint64_t)windows * (uint64_t)b * (uint64_t)m.rows * 4u : 0;
    if (windows == 1 || (ws.ptr && ws.bytes >= need)) {
        // workgroups resident at once, shared out between the windows; rounded down, since a
        // workgroup past the resident count would start only when another one ends and double
        // the launch's time (4096 x 14336 Q6_K at B = 16: 518 workgroups for 512 slots took
        // 31 us)
        constexpr int lds = mfma_lds<FMT, BB>();
        const int measured = g_mfma_resident[fmt_slot(FMT)][bb_slot(BB)];
        const int per_cu = measured > 0 ? measured : (163840 / lds > 0 ? 163840 / lds : 1);
        int grid = g_cus * (per_cu < 8 ? per_cu : 8) / windows;
        if (grid < 1) grid = 1;
        if (grid > tiles) grid = tiles;
        // With rounds of 4 tiles (8 waves, up to 8 rows) and at 16 rows, workgroups with at
        // least one full round take the tile loop without skip paths: A/B on one box, decode
        // step B = 4 1.853 -> 1.818 ms, B = 8 2.110 -> 2.047 ms, B = 16 (with the prologue's
        // tiles loaded in order) 2.443 -> 2.399 ms. With fewer tiles its loads for absent
        // tiles cost more than it saves (Q8_0 4096 x 4096 at B = 4: 9.8 -> 10.6 us), and for
        // Q4_0 and Q8_0 at up to 8 rows (16 waves, rounds of 2) it lost too (Q4_0 11008 x
        // 4096 at B = 8 12.7 -> 13.0 us).
        constexpr int RT = gmf::round_tiles<BB, W>();
        hipError_t e;
        if constexpr (RT >= 4 || BB > 8) {
            if ((tiles + grid - 1) / grid >= RT)
                e = gmf::launch_k<FMT, BB, W, IPW, false, mfma_ring<FMT, BB>(), true>(
                    m, x, windows == 1 ? add : nullptr, y, b, grid, s, 0, per, nb, nullptr, windows, ws.ptr);
            else
                e = gmf::launch_k<FMT, BB, W, IPW, false, mfma_ring<FMT, BB>()>(
                    m, x, windows == 1 ? add : nullptr, y, b, grid, s, 0, per, nb, nullptr, windows, ws.ptr);
        } else {
            e = gmf::launch_k<FMT, BB, W, IPW, false, mfma_ring<FMT, BB>()>(m, x, windows == 1 ? add : nullptr, y, b, grid,
                                                                             s, 0, per, nb, nullptr, windows, ws.ptr);
        }
        if (e != hipSuccess || windows == 1) return e;
        const int64_t n = (int64_t)b * m.rows;
        const int64_t blocks = ((n % 4 == 0 ? n / 4 : n) + 255) / 256;  // a thread per float4 where n allows
        gmf::sum_windows_kernel<<<(unsigned)(blocks < 2048 ? blocks : 2048), 256, 0, s>>>(ws.ptr, windows, n, add, y);
        return hipGetLastError();
    }
    const int grid = tiles < g_cus ? tiles : g_cus;
    for (int kb0 = 0; kb0 < nb; kb0 += per) {
        const bool last = kb0 + per >= nb;
        const hipError_t e = gmf::launch_k<FMT, BB, W, IPW, false, mfma_ring<FMT, BB>()>(m, x, last ? add : nullptr, y, b, grid, s, kb0, per,
                                                                        last ? nb : kb0 + per, kb0 == 0 ? nullptr : y, 1,
                                                                        nullptr);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int FMT>
hipError_t launch_mfma_fmt(const QMat &m, const float *x, const float *add, float *y, int b, const Workspace &ws,
                           hipStream_t s) {
    if (b <= 4) return launch_mfma<FMT, 4>(m, x, add, y, b, ws, s);
    if (b <= 8) return launch_mfma<FMT, 8>(m, x, add, y, b, ws, s);
    return launch_mfma<FMT, 16>(m, x, add, y, b, ws, s);
}

template <int FMT>
uint64_t mfma_ws_fmt(const QMat &m, int b) {
    int windows = 1, per = 0;
    if (b <= 4) mfma_windows<FMT, 4>(m, windows, per);
    else if (b <= 8) mfma_windows<FMT, 8>(m, windows, per);
    else mfma_windows<FMT, 16>(m, windows, per);
    return windows > 1 ? (uint64_t)windows * (uint64_t)b * (uint64_t)m.rows * 4u : 0;
}

uint64_t mfma_ws_any(int id, const QMat &m, int b) {
    switch (id) {
    case Q4_0: return mfma_ws_fmt<Q4_0>(m, b);
    case Q4_K: return mfma_ws_fmt<Q4_K>(m, b);
    case Q6_K: return mfma_ws_fmt<Q6_K>(m, b);
    case Q8_0: return mfma_ws_fmt<Q8_0>(m, b);
    default: return 0;
    }
}

// Several windows read add only in the last one, after y was rewritten: an add that
// overlaps y then keeps a single window (or the single-pass vector-ALU kernel).
template <int BB>
bool single_window(const QMat &m) { return m.cols <= 32 * mfma_window<Q4_0, BB>(); }

bool mfma_format(int id, const QMat &m) {
    const int64_t k = m.cols;
    switch (id) {
    case Q4_0: case Q4_K: case Q6_K: return k % 128 == 0;
    case Q8_0: return k % 64 == 0;
    default: return false;
    }
}

hipError_t launch_mfma_any(int id, const QMat &m, const float *x, const float *add, float *y, int b, const Workspace &ws,
                           hipStream_t s) {
    switch (id) {
    case Q4_0: return launch_mfma_fmt<Q4_0>(m, x, add, y, b, ws, s);
    case Q4_K: return launch_mfma_fmt<Q4_K>(m, x, add, y, b, ws, s);
    case Q6_K: return launch_mfma_fmt<Q6_K>(m, x, add, y, b, ws, s);
    case Q8_0: return launch_mfma_fmt<Q8_0>(m, x, add, y, b, ws, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_valu(int id, const QMat &m, const float *x, const float *add, float *y, int b, hipStream_t s) {
    switch (id) {
    case Q4_0: return launch_fmt<Q4_0>(m, x, add, y, b, g_cus, s);
    case Q8_0: return launch_fmt<Q8_0>(m, x, add, y, b, g_cus, s);
    case Q4_K: return launch_fmt<Q4_K>(m, x, add, y, b, g_cus, s);
    case Q6_K: return launch_fmt<Q6_K>(m, x, add, y, b, g_cus, s);
    case Q2_0: return launch_fmt<Q2_0>(m, x, add, y, b, g_cus, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

void gemv_set_cus(int cus) {
    g_cus = cus > 0 ? cus : 256;
    measure_resident_fmt<Q4_0>();
    measure_resident_fmt<Q8_0>();
    measure_resident_fmt<Q4_K>();
    measure_resident_fmt<Q6_K>();
}

namespace {
std::atomic<int> g_gemv_policy{J4Q_GEMV_MATRIX_CORES};
// whether a batch of `batch` rows runs on the matrix cores
bool on_matrix_cores(int id, const QMat &m, int64_t batch) {
    return batch >= 3 && mfma_format(id, m) && g_gemv_policy.load(std::memory_order_relaxed) == J4Q_GEMV_MATRIX_CORES;
}
}  // namespace

void gemv_set_policy(int policy) { g_gemv_policy.store(policy, std::memory_order_relaxed); }
int gemv_policy() { return g_gemv_policy.load(std::memory_order_relaxed); }

bool gemv_in_place_ok(int id, const QMat &m, int64_t batch) {
    return m.cols <= gemv::kMaxWindow || on_matrix_cores(id, m, batch);
}

uint64_t gemv_workspace_bytes(int id, const QMat &m, int64_t batch) {
    if (m.rows <= 0 || !on_matrix_cores(id, m, batch)) return 0;
    // launches of 16 rows and, for a remainder of 3..15 rows, one smaller launch
    uint64_t need = mfma_ws_any(id, m, (int)(batch < 16 ? batch : 16));
    const int64_t rem = batch % 16;
    if (batch > 16 && rem >= 3) {
        const uint64_t r = mfma_ws_any(id, m, (int)rem);
        if (r > need) need = r;
    }
    if (batch > 16 && (rem == 1 || rem == 2) && m.cols > gemv::kMaxWindow) {
        // launch_gemv then runs 14 or 15 rows (within the 16-row need) and a remainder of 3
        const uint64_t r = mfma_ws_any(id, m, 3);
        if (r > need) need = r;
    }
    return need;
}

hipError_t launch_gemv(int id, const QMat &m, const float *x, const float *add, float *y, int64_t batch,
                       hipStream_t s, const Workspace &ws) {
    if (m.rows <= 0 || batch <= 0) return hipSuccess;
    if (batch > 65535 || m.rows > (1 << 30) || m.cols > 0x7fffffff) return hipErrorInvalidValue;
    const bool alias = add && add < y + batch * m.rows && y < add + batch * m.rows;
    const bool mfma = on_matrix_cores(id, m, batch);
    // with the workspace, several windows meet in sum_windows_kernel, which reads each add
    // element before it writes y there; without it they are chained launches that would
    // read an add overlapping y after rewriting y, so such a call keeps one window
    const bool ws_ok = mfma && ws.ptr && ws.bytes >= gemv_workspace_bytes(id, m, batch);
    if (!mfma || (alias && !ws_ok && !single_window<8>(m))) {
        if (alias && m.cols > gemv::kMaxWindow) return hipErrorInvalidValue;
        return launch_valu(id, m, x, add, y, (int)batch, s);
    }
    // batch rows in launches of up to 16 on the matrix cores (every launch streams W once for
    // its rows); a remainder of 1 or 2 rows takes the vector-ALU kernel, which is as fast there.
    // Above one vector-ALU window (K > 32768) that kernel chains its windows through y, so an
    // add that is y itself would be read after the first window rewrote it: there the last
    // full launch gives up rows so that the remainder makes 3 and stays on the matrix cores
    // (17 -> 14 + 3, 18 -> 15 + 3). In-place and out-of-place calls split the same way, so
    // they agree bit for bit.
    const int64_t cap = !alias || ws_ok || single_window<16>(m) ? 16 : 8;
    const int64_t rem = batch % cap;
    const bool wide = m.cols > gemv::kMaxWindow && batch > cap && (rem == 1 || rem == 2);
    for (int64_t b0 = 0; b0 < batch;) {
        int64_t nb = batch - b0 < cap ? batch - b0 : cap;
        if (wide && batch - b0 == cap + rem) nb = cap + rem - 3;
        const float *xb = x + b0 * m.cols;
        const float *ab = add ? add + b0 * m.rows : nullptr;
        float *yb = y + b0 * m.rows;
        const hipError_t e = nb >= 3 ? launch_mfma_any(id, m, xb, ab, yb, (int)nb, ws_ok ? ws : Workspace(), s)
                                     : launch_valu(id, m, xb, ab, yb, (int)nb, s);
        if (e != hipSuccess) return e;
        b0 += nb;
    }
    return hipSuccess;
}

}  // namespace j4q

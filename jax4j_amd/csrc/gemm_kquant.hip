// Prefill GEMM over Q4_0, Q4_K and Q6_K weights (bf16 variant; kernels in gemm_kquant.h):
// picks the tile and the K split for the shape.
#include "j4q_common.h"
#include "gemm_kquant.h"

namespace j4q {
namespace {

// Launch shape: the largest tile whose grid still fills the GPU (128 x 128 when that makes
// >= 256 workgroups, else 128 x 64), else 64 x 64 tiles (32 x 64 for M <= 32) with K split
// into S ranges of whole stages when there are fewer than 192 tiles, for about 512
// workgroups in all (two or three per CU: each workgroup walks its stages as one dependent
// chain, so a thin grid leaves the CUs waiting on it). The splits' partial products are
// added in order by sum_splits_kernel, so results do not depend on the device; their
// workspace is capped at 32 MiB (no split above it).
struct KqShape {
    int bm, nj, splits, stages;  // tile rows, 64-column tiles, K splits, stages per split
    int64_t tiles;
};

KqShape kq_shape(const QMat &w, int64_t m) {
    const int64_t nt64 = (w.rows + 63) / 64, nt128 = (w.rows + 127) / 128, ns = w.cols / 128;
    KqShape sh{64, 1, 1, (int)ns, 0};
    if (((m + 127) / 128) * nt128 >= 256) {
        sh.bm = 128;
        sh.nj = 2;
        sh.tiles = ((m + 127) / 128) * nt128;
        return sh;
    }
    if (((m + 127) / 128) * nt64 >= 256) {
        sh.bm = 128;
        sh.tiles = ((m + 127) / 128) * nt64;
        return sh;
    }
    sh.bm = m <= 32 ? 32 : 64;
    sh.tiles = ((m + sh.bm - 1) / sh.bm) * nt64;
    if (sh.tiles < 192) {
        int64_t want = (512 + sh.tiles - 1) / sh.tiles;
        if (want > ns / 4) want = ns / 4;  // at least four stages per split
        while (want > 1 && (uint64_t)want * (uint64_t)m * (uint64_t)w.rows * 4u > (32ull << 20)) want--;
        if (want > 1) {
            const int64_t per = (ns + want - 1) / want;
            sh.stages = (int)per;
            sh.splits = (int)((ns + per - 1) / per);
        }
    }
    return sh;
}

template <int FMT, int BM, int NJ>
hipError_t launch_tile(const QMat &w, const uint16_t *x, float *y, int64_t m, const KqShape &sh, float *ws,
                       hipStream_t s) {
    gk::gemm_kq_bf16<FMT, BM, NJ><<<dim3((unsigned)sh.tiles, (unsigned)sh.splits), 512, 0, s>>>(
        w, x, y, (int)m, sh.stages, sh.splits > 1 ? ws : nullptr);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_kq(const QMat &w, const uint16_t *x, float *y, int64_t m, float *ws, hipStream_t s) {
    const KqShape sh = kq_shape(w, m);
    if (sh.tiles > 0x7fffffff) return hipErrorInvalidValue;
    if (sh.splits > 1 && !ws) return hipErrorInvalidValue;
    hipError_t e;
    if (sh.bm == 128) e = sh.nj == 2 ? launch_tile<FMT, 128, 2>(w, x, y, m, sh, ws, s) : launch_tile<FMT, 128, 1>(w, x, y, m, sh, ws, s);
    else if (sh.bm == 64) e = launch_tile<FMT, 64, 1>(w, x, y, m, sh, ws, s);
    else e = launch_tile<FMT, 32, 1>(w, x, y, m, sh, ws, s);
    if (e != hipSuccess || sh.splits == 1) return e;
    const int64_t n = m * w.rows;
    const int64_t blocks = ((n % 4 == 0 ? n / 4 : n) + 255) / 256;
    gk::sum_splits_kernel<<<(unsigned)(blocks < 2048 ? blocks : 2048), 256, 0, s>>>(ws, sh.splits, n, y);
    return hipGetLastError();
}

}  // namespace

bool gemm_kq_supported(int id, int64_t cols) {
    switch (id) {
    case Q4_0: return cols % 128 == 0;
    case Q4_K:
    case Q6_K: return cols % 256 == 0;
    default: return false;
    }
}

uint64_t gemm_kq_workspace_bytes(int id, const QMat &w, int64_t m) {
    if (!gemm_kq_supported(id, w.cols) || m <= 0 || w.rows <= 0) return 0;
    const KqShape sh = kq_shape(w, m);
    return sh.splits > 1 ? (uint64_t)sh.splits * (uint64_t)m * (uint64_t)w.rows * 4u : 0;
}

hipError_t launch_gemm_kq_bf16(int id, const QMat &w, const uint16_t *x, float *y, int64_t m, float *ws,
                               hipStream_t s) {
    if (m <= 0 || w.rows <= 0) return hipSuccess;
    if (!gemm_kq_supported(id, w.cols) || (uint64_t)m * (uint64_t)w.cols * 2u > 0x7fffffffull ||
        (uint64_t)w.rows * (uint64_t)w.cols / 2u > 0x7fffffffull)
        return hipErrorInvalidValue;
    switch (id) {
    case Q4_0: return launch_kq<Q4_0>(w, x, y, m, ws, s);
    case Q4_K: return launch_kq<Q4_K>(w, x, y, m, ws, s);
    case Q6_K: return launch_kq<Q6_K>(w, x, y, m, ws, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace j4q

// Prefill GEMM over Q4_0, Q4_K and Q6_K weights (bf16 variant; kernels in gemm_kquant.h):
// picks the tile for the shape.
#include "j4q_common.h"
#include "gemm_kquant.h"

namespace j4q {
namespace {

// The largest tile whose grid still fills the GPU: 128 x 128 when that makes >= 256
// workgroups, else 128 x 64, else 64 x 64 (two workgroups per CU).
template <int FMT>
hipError_t launch_kq(const QMat &w, const uint16_t *x, float *y, int64_t m, hipStream_t s) {
    const int64_t nt128 = (w.rows + 127) / 128, nt64 = (w.rows + 63) / 64;
    const int64_t g128x128 = ((m + 127) / 128) * nt128, g128x64 = ((m + 127) / 128) * nt64, g64 = ((m + 63) / 64) * nt64;
    if (g64 > 0x7fffffff) return hipErrorInvalidValue;
    if (g128x128 >= 256)
        gk::gemm_kq_bf16<FMT, 128, 2><<<(unsigned)g128x128, 512, 0, s>>>(w, x, y, (int)m);
    else if (g128x64 >= 256)
        gk::gemm_kq_bf16<FMT, 128, 1><<<(unsigned)g128x64, 512, 0, s>>>(w, x, y, (int)m);
    else
        gk::gemm_kq_bf16<FMT, 64, 1><<<(unsigned)g64, 512, 0, s>>>(w, x, y, (int)m);
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

hipError_t launch_gemm_kq_bf16(int id, const QMat &w, const uint16_t *x, float *y, int64_t m, hipStream_t s) {
    if (m <= 0 || w.rows <= 0) return hipSuccess;
    if (!gemm_kq_supported(id, w.cols) || (uint64_t)m * (uint64_t)w.cols * 2u > 0x7fffffffull ||
        (uint64_t)w.rows * (uint64_t)w.cols / 2u > 0x7fffffffull)
        return hipErrorInvalidValue;
    switch (id) {
    case Q4_0: return launch_kq<Q4_0>(w, x, y, m, s);
    case Q4_K: return launch_kq<Q4_K>(w, x, y, m, s);
    case Q6_K: return launch_kq<Q6_K>(w, x, y, m, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace j4q

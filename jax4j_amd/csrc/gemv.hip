// Decode GEMV dispatch: picks the row-group size R, waves per workgroup and grid size of
// the persistent GEMV kernel (gemv_impl.h) for each format and shape.
#include "gemv_impl.h"

namespace j4q {

// Largest K whose x image (K floats + K/16 sums) fits the 64 KiB of LDS a workgroup may use.
int64_t gemv_max_cols() { return 15360; }

namespace {

// Launch shape, from measured sweeps on MI355X (one row per group, two register sets in
// flight): for K <= 8192, 8 waves per workgroup and 2 workgroups per CU; for larger K (an
// x image of up to 64 KiB), 16 waves in one workgroup per CU. The grid never exceeds what
// is resident at once, so x is staged once per workgroup.
template <int FMT>
hipError_t launch_fmt(const QMat &m, const float *x, const float *add, float *y, int batch, int cus,
                      hipStream_t s) {
    if (m.cols <= 8192) return gemv::launch<FMT, 1, 8, 2>(m, x, add, y, batch, 2 * cus, s);
    return gemv::launch<FMT, 1, 16, 2>(m, x, add, y, batch, cus, s);
}

int g_cus = 256;

}  // namespace

void gemv_set_cus(int cus) { g_cus = cus > 0 ? cus : 256; }

hipError_t launch_gemv(int id, const QMat &m, const float *x, const float *add, float *y, int64_t batch,
                       hipStream_t s) {
    if (m.rows <= 0 || batch <= 0) return hipSuccess;
    if (m.cols > gemv_max_cols() || batch > 65535 || m.rows > (1 << 30)) return hipErrorInvalidValue;
    const int b = (int)batch;
    switch (id) {
    case Q4_0: return launch_fmt<Q4_0>(m, x, add, y, b, g_cus, s);
    case Q8_0: return launch_fmt<Q8_0>(m, x, add, y, b, g_cus, s);
    case Q4_K: return launch_fmt<Q4_K>(m, x, add, y, b, g_cus, s);
    case Q6_K: return launch_fmt<Q6_K>(m, x, add, y, b, g_cus, s);
    case Q2_0: return launch_fmt<Q2_0>(m, x, add, y, b, g_cus, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace j4q

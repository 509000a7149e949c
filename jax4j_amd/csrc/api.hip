// C ABI of the engine (declared in include/jax4j_mi355x.h): buffer table, argument checks,
// error reporting and dispatch to the kernels. Every argument check happens before the
// first HIP call, so all error paths can be exercised on a machine without a GPU.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "engine.h"
#include "synth.h"

namespace j4q {
int64_t gemv_single_pass_cols();
void gemv_set_cus(int cus);
void gemv_set_trace(uint64_t *words, int64_t n);
}

namespace {

using j4q::Geometry;

struct Buf {
    int kind = 0;
    int qtype = 0;
    int rank = 0;
    int64_t dims[2] = {0, 0};
    void *dev = nullptr;
    uint64_t bytes = 0;
    uint32_t gen = 0;
    bool live = false;
    // decode plans whose captured graph reads this buffer's memory; while any lives the
    // buffer cannot be released (last_plan names one of them in the error)
    int32_t pins = 0;
    uint64_t last_plan = 0;
};

// Workspace of j4q_quant_matmul_noalloc (the one entry point that allocates nothing): the
// int8 activations [m, K] of one call in the first 32 MiB, their fp32 block scales
// [m, K / 32] (at most 4 MiB for m * K <= 32 MiB) after them. Every GPU the library runs on
// holds its own copy until the process ends; host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address) but the address
// hipGetSymbolAddress returns for the engine's device, kept in g_scratch. Calls that overlap
// on one GPU share it and race.
constexpr uint64_t kScratchQBytes = 32ull << 20;
constexpr uint64_t kScratchBytes = kScratchQBytes + (4ull << 20);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
std::vector<Buf> g_bufs;
void *g_scratch = nullptr;  // device address of `scratch` on g_dev
std::vector<uint32_t> g_free;
bool g_ready = false;
int g_dev = -1;
hipStream_t g_stream = nullptr;
thread_local std::string t_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

int hip_fail(const char *op, hipError_t e) { return j4q::report_hip(op, e); }

#define HIP_TRY(op, expr)                         \
    do {                                          \
        hipError_t e_ = (expr);                   \
        if (e_ != hipSuccess) return hip_fail(op, e_); \
    } while (0)

}  // namespace

namespace j4q {
// Error reporting for the other translation units: same thread-local message as every entry point.
int report_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

int report_hip(const char *op, hipError_t e) {
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? J4Q_ENOMEM : J4Q_EHIP;
    return report_error(code, "%s failed: %s (code %d)", op, hipGetErrorString(e), (int)e);
}
}  // namespace j4q

namespace {

bool is_gfx950(const hipDeviceProp_t &p) { return strncmp(p.gcnArchName, "gfx950", 6) == 0; }

// Requires g_mu held.
int ensure_ready() {
    if (g_ready) {
        HIP_TRY("hipSetDevice", hipSetDevice(g_dev));
        return J4Q_OK;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(J4Q_ENODEV, "no HIP device is available");
    return fail(J4Q_ENODEV, "engine not initialised: call j4q_init first");
}

int init_locked(int device) {
    if (g_ready) {
        if (device != g_dev) return fail(J4Q_EINVAL, "engine already initialised on device %d, not %d", g_dev, device);
        HIP_TRY("hipSetDevice", hipSetDevice(g_dev));
        return J4Q_OK;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(J4Q_ENODEV, "no HIP device is available");
    if (device < 0 || device >= n) return fail(J4Q_EINVAL, "device %d out of range [0, %d)", device, n);
    hipDeviceProp_t p;
    HIP_TRY("hipGetDeviceProperties", hipGetDeviceProperties(&p, device));
    if (!is_gfx950(p)) return fail(J4Q_ENODEV, "device %d is %s; this engine is built for gfx950 only", device, p.gcnArchName);
    HIP_TRY("hipSetDevice", hipSetDevice(device));
    // the engine serves one device per process, so one address of the workspace is kept
    HIP_TRY("hipGetSymbolAddress", hipGetSymbolAddress(&g_scratch, HIP_SYMBOL(scratch)));
    HIP_TRY("hipStreamCreateWithFlags", hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    j4q::gemv_set_cus(p.multiProcessorCount);
    g_dev = device;
    g_ready = true;
    return J4Q_OK;
}

j4q_buffer make_handle(uint32_t slot, uint32_t gen) { return ((uint64_t)gen << 32) | (uint64_t)(slot + 1); }

Buf *lookup(j4q_buffer h) {
    const uint64_t lo = h & 0xffffffffu;
    if (lo == 0 || lo > g_bufs.size()) return nullptr;
    Buf &b = g_bufs[lo - 1];
    if (!b.live || b.gen != (uint32_t)(h >> 32)) return nullptr;
    return &b;
}

j4q_buffer register_buf(const Buf &nb) {
    uint32_t slot;
    if (!g_free.empty()) {
        slot = g_free.back();
        g_free.pop_back();
    } else {
        slot = (uint32_t)g_bufs.size();
        g_bufs.emplace_back();
    }
    const uint32_t gen = g_bufs[slot].gen + 1;
    g_bufs[slot] = nb;
    g_bufs[slot].gen = gen;
    g_bufs[slot].live = true;
    return make_handle(slot, gen);
}

int get_buf(j4q_buffer h, int kind, const char *what, Buf **out) {
    Buf *b = lookup(h);
    if (!b) return fail(J4Q_EHANDLE, "%s: unknown or released buffer handle 0x%llx", what, (unsigned long long)h);
    if (kind && b->kind != kind) return fail(J4Q_EHANDLE, "%s: buffer 0x%llx has the wrong kind (%d, expected %d)", what, (unsigned long long)h, b->kind, kind);
    *out = b;
    return J4Q_OK;
}

int64_t elements_of(const Buf &b) { return b.rank == 1 ? b.dims[0] : b.dims[0] * b.dims[1]; }

// Allocates a device buffer of `bytes` (0 allowed) and registers it.
// Registering may grow the buffer table, so callers keep the returned device pointer, not
// a Buf* taken before the call.
int alloc_buf(int kind, int rank, int64_t d0, int64_t d1, uint64_t bytes, j4q_buffer *out, void **dev_out) {
    Buf nb;
    nb.kind = kind;
    nb.rank = rank;
    nb.dims[0] = d0;
    nb.dims[1] = d1;
    nb.bytes = bytes;
    if (bytes) HIP_TRY("hipMalloc", hipMalloc(&nb.dev, bytes));
    *out = register_buf(nb);
    *dev_out = nb.dev;
    return J4Q_OK;
}

// Undoes alloc_buf after a failed launch: frees the memory, retires the handle and clears
// *out, so a rejected call leaves no live buffer behind.
void drop_buf(j4q_buffer *out) {
    Buf *b = lookup(*out);
    if (b) {
        if (b->dev) (void)hipFree(b->dev);
        b->dev = nullptr;
        b->live = false;
        g_free.push_back((uint32_t)((*out & 0xffffffffu) - 1));
    }
    *out = 0;
}

// Launches into a buffer alloc_buf just registered; on failure the buffer is dropped again.
#define LAUNCH_INTO(op, out, expr)                 \
    do {                                           \
        hipError_t e_ = (expr);                    \
        if (e_ != hipSuccess) {                    \
            drop_buf(out);                         \
            return hip_fail(op, e_);               \
        }                                          \
    } while (0)

int check_quant_args(int qt, uint64_t nbytes, int64_t rows, int64_t cols, Geometry *g) {
    if (!j4q::geometry_of(qt, g)) {
        const int known[] = {0, 1, 2, 8, 12, 14, 30, 41, 42};
        for (int k : known)
            if (k == qt) return fail(J4Q_EUNSUPPORTED, "unsupported quant type id %d", qt);
        return fail(J4Q_EINVAL, "unknown ggml quant type id: %d", qt);
    }
    if (rows <= 0 || cols <= 0 || cols % g->block_elements != 0)
        return fail(J4Q_EINVAL, "invalid quantized matrix dimensions: rows=%lld cols=%lld block=%d", (long long)rows,
                    (long long)cols, g->block_elements);
    const int64_t blocks_per_row = cols / g->block_elements;
    if (rows > INT64_MAX / blocks_per_row || rows * blocks_per_row > INT64_MAX / g->block_bytes)
        return fail(J4Q_EINVAL, "quantized matrix too large: rows=%lld cols=%lld", (long long)rows, (long long)cols);
    const uint64_t need = (uint64_t)(rows * blocks_per_row) * (uint64_t)g->block_bytes;
    if (nbytes != need)
        return fail(J4Q_EINVAL, "quantized blob is %llu bytes, expected %llu for [%lld, %lld]", (unsigned long long)nbytes,
                    (unsigned long long)need, (long long)rows, (long long)cols);
    return J4Q_OK;
}

// The kernels address each section of a resident matrix with 32-bit buffer offsets.
int check_sections(int qt, int64_t rows, int64_t cols) {
    const j4q::SplitLayout L = j4q::split_layout(qt, rows, cols);
    const uint64_t lim = 0x7fffffffull;
    if (L.qs_bytes > lim || L.qh_bytes > lim || L.sc_bytes > lim || L.d_bytes > lim || rows > (1 << 30))
        return fail(J4Q_EUNSUPPORTED, "quantized matrix [%lld, %lld] exceeds 2 GiB per section", (long long)rows,
                    (long long)cols);
    return J4Q_OK;
}

int upload_quant_common(int qt, const void *src, bool src_on_device, uint64_t nbytes, int64_t rows, int64_t cols,
                        j4q_buffer *out) {
    Geometry g;
    if (!src) return fail(J4Q_EINVAL, "uploadQuantized: blocks is NULL");
    if (!out) return fail(J4Q_EINVAL, "uploadQuantized: out is NULL");
    int rc = check_quant_args(qt, nbytes, rows, cols, &g);
    if (rc) return rc;
    if ((rc = check_sections(qt, rows, cols))) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    if ((rc = ensure_ready())) return rc;
    const j4q::SplitLayout L = j4q::split_layout(qt, rows, cols);
    void *staging = nullptr;
    const void *gguf = src;
    if (!src_on_device) {
        HIP_TRY("hipMalloc", hipMalloc(&staging, nbytes));
        hipError_t e = hipMemcpyAsync(staging, src, nbytes, hipMemcpyHostToDevice, g_stream);
        if (e != hipSuccess) {
            (void)hipFree(staging);
            return hip_fail("hipMemcpyAsync", e);
        }
        gguf = staging;
    }
    void *dev = nullptr;
    hipError_t e = hipMalloc(&dev, L.total);
    if (e == hipSuccess) e = j4q::launch_repack(qt, (const uint8_t *)gguf, (uint8_t *)dev, rows, cols, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        if (dev) (void)hipFree(dev);
        return hip_fail("uploadQuantized", e);
    }
    Buf nb;
    nb.kind = J4Q_KIND_QUANT;
    nb.qtype = qt;
    nb.rank = 2;
    nb.dims[0] = rows;
    nb.dims[1] = cols;
    nb.dev = dev;
    nb.bytes = L.total;
    *out = register_buf(nb);
    return J4Q_OK;
}

int upload_dense(int kind, int elem_bytes, const void *data, int32_t rank, const int64_t *dims, j4q_buffer *out) {
    if (!out || !dims) return fail(J4Q_EINVAL, "upload: NULL argument");
    if (rank != 1 && rank != 2) return fail(J4Q_EINVAL, "upload: rank %d not supported (1 or 2)", rank);
    const int64_t d0 = dims[0], d1 = rank == 2 ? dims[1] : 1;
    if (d0 < 0 || d1 < 0) return fail(J4Q_EINVAL, "upload: negative dimension");
    if (d1 && d0 > INT64_MAX / d1 / elem_bytes) return fail(J4Q_EINVAL, "upload: shape too large");
    const uint64_t bytes = (uint64_t)(d0 * d1) * elem_bytes;
    if (bytes && !data) return fail(J4Q_EINVAL, "upload: data is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    void *dev = nullptr;
    if ((rc = alloc_buf(kind, rank, d0, rank == 2 ? d1 : 0, bytes, out, &dev))) return rc;
    if (bytes) {
        hipError_t e = hipMemcpyAsync(dev, data, bytes, hipMemcpyHostToDevice, g_stream);
        if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
        if (e != hipSuccess) {
            drop_buf(out);
            return hip_fail("upload", e);
        }
    }
    return J4Q_OK;
}

j4q::QMat qmat_of(const Buf &w) {
    return j4q::qmat_view((const uint8_t *)w.dev, w.qtype, w.dims[0], w.dims[1]);
}

// Shape rule of quantMatvec (CpuBackend.java:712): x must hold exactly cols values; the
// engine also accepts [B, cols] for B > 1. Returns batch or -1.
int64_t matvec_batch(const Buf &w, const Buf &x) {
    const int64_t K = w.dims[1];
    if (elements_of(x) == K) return 1;
    if (x.rank == 2 && x.dims[1] == K && x.dims[0] > 1) return x.dims[0];
    return -1;
}

int matvec_common(j4q_buffer wh, j4q_buffer xh, j4q_buffer addh, j4q_buffer *out, const char *op) {
    if (!out) return fail(J4Q_EINVAL, "%s: out is NULL", op);
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w, *x, *add = nullptr;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, op, &w))) return rc;
    if ((rc = get_buf(xh, J4Q_KIND_F32, op, &x))) return rc;
    if (addh && (rc = get_buf(addh, J4Q_KIND_F32, op, &add))) return rc;
    const int64_t B = matvec_batch(*w, *x);
    if (B < 0)
        return fail(J4Q_EINVAL, "%s shape mismatch: [%lld, %lld] x [%lld%s%lld]", op, (long long)w->dims[0],
                    (long long)w->dims[1], (long long)x->dims[0], x->rank == 2 ? ", " : "",
                    x->rank == 2 ? (long long)x->dims[1] : 0LL);
    const int64_t N = w->dims[0];
    if (add && elements_of(*add) < B * N)
        return fail(J4Q_EINVAL, "%s: add has %lld elements, needs %lld", op, (long long)elements_of(*add), (long long)(B * N));
    if (B > 65535) return fail(J4Q_EUNSUPPORTED, "%s: batch %lld exceeds 65535", op, (long long)B);
    if ((rc = ensure_ready())) return rc;
    const void *xdev = x->dev, *adev = add ? add->dev : nullptr;
    const j4q::QMat m = qmat_of(*w);
    const int qt = w->qtype;
    void *ydev;
    if ((rc = alloc_buf(J4Q_KIND_F32, B == 1 ? 1 : 2, B == 1 ? N : B, B == 1 ? 0 : N, (uint64_t)(B * N) * 4, out, &ydev)))
        return rc;
    // a batched call over several column windows runs them in one launch on a stream-ordered
    // workspace for their partial sums; if it cannot be had, the windows run one after another
    j4q::Workspace ws;
    const uint64_t wsb = j4q::gemv_workspace_bytes(qt, m, B);
    if (wsb) {
        void *p = nullptr;
        if (hipMallocAsync(&p, wsb, g_stream) == hipSuccess) {
            ws.ptr = (float *)p;
            ws.bytes = wsb;
        } else {
            (void)hipGetLastError();
        }
    }
    const hipError_t e = j4q::launch_gemv(qt, m, (const float *)xdev, (const float *)adev, (float *)ydev, B, g_stream, ws);
    if (ws.ptr) (void)hipFreeAsync(ws.ptr, g_stream);
    LAUNCH_INTO(op, out, e);
    return J4Q_OK;
}

// Size limits of the prefill GEMM kernels (32-bit element offsets into X and W, grid
// dimensions), checked before anything is allocated.
int check_gemm_size(int64_t M, int64_t K, int variant, const char *op) {
    const uint64_t xbytes = (uint64_t)M * (uint64_t)K * (variant == J4Q_GEMM_BF16 ? 2u : 1u);
    if (M > 65535 * 64 || xbytes > 0x7fffffffull)
        return fail(J4Q_EUNSUPPORTED, "%s: M = %lld, K = %lld exceeds the GEMM limits (M <= %d, X under 2 GiB)", op,
                    (long long)M, (long long)K, 65535 * 64);
    return J4Q_OK;
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

hipStream_t pick_stream(void *s) { return s ? (hipStream_t)s : g_stream; }

// Weight types of the prefill GEMM: Q8_0 for both variants; Q4_0 (cols % 128 == 0), Q4_K
// and Q6_K for the bf16 variant (the int8 variant folds one Q8_0 scale per 32-block).
int check_gemm_weights(const Buf &w, int variant, const char *op) {
    if (w.qtype == J4Q_Q8_0) return J4Q_OK;
    if (variant == J4Q_GEMM_INT8)
        return fail(J4Q_EUNSUPPORTED, "%s: the int8 variant needs Q8_0 weights, got type %d (use the bf16 variant)", op,
                    w.qtype);
    if (!j4q::gemm_kq_supported(w.qtype, w.dims[1]))
        return fail(J4Q_EUNSUPPORTED, "%s: no GEMM for type %d with %lld columns (Q8_0, Q4_0 with cols %% 128 == 0, Q4_K, Q6_K)",
                    op, w.qtype, (long long)w.dims[1]);
    return J4Q_OK;
}

// Takes the weight type by value: callers read it before alloc_buf, whose registration of the
// output can move the buffer table (and every Buf pointer into it).
hipError_t launch_gemm_bf16(int qtype, const j4q::QMat &m, const uint16_t *x, float *y, int64_t rows, float *ws,
                            hipStream_t s) {
    return qtype == J4Q_Q8_0 ? j4q::launch_gemm_q8_bf16(m, x, y, rows, s) : j4q::launch_gemm_kq_bf16(qtype, m, x, y, rows, ws, s);
}

// Workspace of a bf16 GEMM (the K-quant kernels' split partials; none for Q8_0), at most
// 32 MiB.
uint64_t gemm_bf16_workspace(int qtype, const j4q::QMat &m, int64_t rows) {
    return qtype == J4Q_Q8_0 ? 0 : j4q::gemm_kq_workspace_bytes(qtype, m, rows);
}

}  // namespace

namespace j4q {
namespace abi {

std::mutex &lock() { return g_mu; }
int ready_locked() { return ensure_ready(); }
hipStream_t stream() { return g_stream; }

int quant_locked(j4q_buffer h, const char *op, QuantRef *out) {
    Buf *b;
    const int rc = get_buf(h, J4Q_KIND_QUANT, op, &b);
    if (rc) return rc;
    Geometry g;
    geometry_of(b->qtype, &g);
    out->qtype = b->qtype;
    out->rows = b->dims[0];
    out->cols = b->dims[1];
    out->m = qmat_of(*b);
    out->gguf_bytes = (uint64_t)(b->dims[0] * (b->dims[1] / g.block_elements)) * (uint64_t)g.block_bytes;
    return J4Q_OK;
}

int pin_locked(j4q_buffer h, uint64_t plan) {
    Buf *b = lookup(h);
    if (!b) return fail(J4Q_EHANDLE, "decode plan: buffer 0x%llx was released", (unsigned long long)h);
    b->pins++;
    b->last_plan = plan;
    return J4Q_OK;
}

void unpin_locked(j4q_buffer h) {
    Buf *b = lookup(h);
    if (b && b->pins > 0) b->pins--;
}

int concat_locked(const j4q_buffer *parts, int count, void **dev_out, QuantRef *out) {
    if (count < 1 || count > 64) return fail(J4Q_EINVAL, "concat_rows: count %d out of range [1, 64]", count);
    int rc;
    std::vector<Buf *> ps((size_t)count);
    int64_t rows = 0;
    for (int i = 0; i < count; i++) {
        if ((rc = get_buf(parts[i], J4Q_KIND_QUANT, "concat_rows", &ps[(size_t)i]))) return rc;
        if (ps[(size_t)i]->qtype != ps[0]->qtype || ps[(size_t)i]->dims[1] != ps[0]->dims[1])
            return fail(J4Q_EINVAL, "concat_rows: part %d is type %d with %lld columns; part 0 is type %d with %lld", i,
                        ps[(size_t)i]->qtype, (long long)ps[(size_t)i]->dims[1], ps[0]->qtype, (long long)ps[0]->dims[1]);
        rows += ps[(size_t)i]->dims[0];
    }
    const int qt = ps[0]->qtype;
    const int64_t cols = ps[0]->dims[1];
    if ((rc = check_sections(qt, rows, cols))) return rc;
    if ((rc = ensure_ready())) return rc;
    // every row-major section of the split layout lands at the part's row offset in the
    // matching section of the result; Q8_0's block-major scale copy is rebuilt afterwards
    const SplitLayout L = split_layout(qt, rows, cols);
    void *dev = nullptr;
    HIP_TRY("hipMalloc", hipMalloc(&dev, L.total));
    hipError_t e = hipSuccess;
    uint64_t off[4] = {0, 0, 0, 0};
    for (int i = 0; i < count && e == hipSuccess; i++) {
        const Buf &b = *ps[(size_t)i];
        const SplitLayout P = split_layout(qt, b.dims[0], cols);
        const uint64_t src_off[4] = {P.qs_off, P.qh_off, P.sc_off, P.d_off};
        const uint64_t dst_off[4] = {L.qs_off, L.qh_off, L.sc_off, L.d_off};
        const uint64_t len[4] = {P.qs_bytes, P.qh_bytes, P.sc_bytes, qt == Q8_0 ? 0 : P.d_bytes};
        for (int sct = 0; sct < 4 && e == hipSuccess; sct++) {
            if (!len[sct]) continue;
            e = hipMemcpyAsync((uint8_t *)dev + dst_off[sct] + off[sct], (const uint8_t *)b.dev + src_off[sct], len[sct],
                               hipMemcpyDeviceToDevice, g_stream);
            off[sct] += len[sct];
        }
    }
    if (e == hipSuccess && qt == Q8_0) e = launch_q8_scales_t(qmat_view((const uint8_t *)dev, qt, rows, cols), g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail("concat_rows", e);
    }
    Geometry g;
    geometry_of(qt, &g);
    out->qtype = qt;
    out->rows = rows;
    out->cols = cols;
    out->m = qmat_view((const uint8_t *)dev, qt, rows, cols);
    out->gguf_bytes = (uint64_t)(rows * (cols / g.block_elements)) * (uint64_t)g.block_bytes;
    *dev_out = dev;
    return J4Q_OK;
}

}  // namespace abi
}  // namespace j4q

extern "C" {

int j4q_abi_version(void) { return J4Q_ABI_VERSION; }

int j4q_probe(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    for (int d = 0; d < n; d++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, d) == hipSuccess && is_gfx950(p)) return 1;
    }
    return 0;
}

int j4q_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return init_locked(device);
}

const char *j4q_last_error(void) { return t_err.c_str(); }

int j4q_device_info(j4q_device_props *out) {
    if (!out) return fail(J4Q_EINVAL, "device_info: out is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    hipDeviceProp_t p;
    HIP_TRY("hipGetDeviceProperties", hipGetDeviceProperties(&p, g_dev));
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s", p.name);
    snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->device = g_dev;
    out->compute_units = p.multiProcessorCount;
    out->max_clock_khz = p.clockRate;
    out->l2_bytes = p.l2CacheSize;
    out->hbm_bytes = p.totalGlobalMem;
    return J4Q_OK;
}

int j4q_sync(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    HIP_TRY("hipStreamSynchronize", hipStreamSynchronize(g_stream));
    return J4Q_OK;
}

int j4q_stream(void **out_stream) {
    if (!out_stream) return fail(J4Q_EINVAL, "stream: out is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    *out_stream = (void *)g_stream;
    return J4Q_OK;
}

int j4q_quant_type_info(int qt, int32_t *be, int32_t *bb) {
    Geometry g;
    if (!j4q::geometry_of(qt, &g)) return fail(J4Q_EUNSUPPORTED, "unsupported quant type id %d", qt);
    if (be) *be = g.block_elements;
    if (bb) *bb = g.block_bytes;
    return J4Q_OK;
}

int j4q_quant_byte_size(int qt, int64_t elements, uint64_t *out_bytes) {
    Geometry g;
    if (!j4q::geometry_of(qt, &g)) return fail(J4Q_EUNSUPPORTED, "unsupported quant type id %d", qt);
    if (!out_bytes) return fail(J4Q_EINVAL, "byte_size: out is NULL");
    if (elements < 0 || elements % g.block_elements != 0)
        return fail(J4Q_EINVAL, "tensor is not block-aligned: %lld elements, block=%d", (long long)elements, g.block_elements);
    const int64_t blocks = elements / g.block_elements;
    if (blocks > INT64_MAX / g.block_bytes) return fail(J4Q_EINVAL, "byte size overflows: %lld elements", (long long)elements);
    *out_bytes = (uint64_t)(blocks * g.block_bytes);
    return J4Q_OK;
}

int j4q_supported_quant_types(int32_t *ids, int32_t capacity, int32_t *count) {
    static const int32_t kIds[] = {J4Q_Q2_0, J4Q_Q4_0, J4Q_Q8_0, J4Q_Q4_K, J4Q_Q6_K};
    const int32_t n = (int32_t)(sizeof kIds / sizeof kIds[0]);
    if (!count) return fail(J4Q_EINVAL, "supported_quant_types: count is NULL");
    if (capacity > 0 && !ids) return fail(J4Q_EINVAL, "supported_quant_types: ids is NULL");
    for (int32_t i = 0; i < n && i < capacity; i++) ids[i] = kIds[i];
    *count = n;
    return J4Q_OK;
}

int j4q_upload_quantized(int qt, const void *blocks, uint64_t nbytes, int64_t rows, int64_t cols, j4q_buffer *out) {
    return upload_quant_common(qt, blocks, false, nbytes, rows, cols, out);
}

int j4q_upload_quantized_device(int qt, const void *dblocks, uint64_t nbytes, int64_t rows, int64_t cols,
                                j4q_buffer *out) {
    return upload_quant_common(qt, dblocks, true, nbytes, rows, cols, out);
}

int j4q_export_quantized(j4q_buffer wh, void *blocks, uint64_t nbytes) {
    if (!blocks) return fail(J4Q_EINVAL, "export: blocks is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "export", &w))) return rc;
    Geometry g;
    j4q::geometry_of(w->qtype, &g);
    const uint64_t need = (uint64_t)(w->dims[0] * (w->dims[1] / g.block_elements)) * g.block_bytes;
    if (nbytes != need) return fail(J4Q_EINVAL, "export: buffer is %llu bytes, need %llu", (unsigned long long)nbytes, (unsigned long long)need);
    if ((rc = ensure_ready())) return rc;
    void *tmp = nullptr;
    HIP_TRY("hipMalloc", hipMalloc(&tmp, need));
    hipError_t e = j4q::launch_export(w->qtype, (const uint8_t *)w->dev, (uint8_t *)tmp, w->dims[0], w->dims[1], g_stream);
    if (e == hipSuccess) e = hipMemcpyAsync(blocks, tmp, need, hipMemcpyDeviceToHost, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail("export", e);
    return J4Q_OK;
}

int j4q_concat_rows(const j4q_buffer *parts, int32_t count, j4q_buffer *out) {
    if (!parts || !out) return fail(J4Q_EINVAL, "concat_rows: NULL argument");
    std::lock_guard<std::mutex> lk(g_mu);
    void *dev = nullptr;
    j4q::abi::QuantRef r;
    int rc = j4q::abi::concat_locked(parts, count, &dev, &r);
    if (rc) return rc;
    Buf nb;
    nb.kind = J4Q_KIND_QUANT;
    nb.qtype = r.qtype;
    nb.rank = 2;
    nb.dims[0] = r.rows;
    nb.dims[1] = r.cols;
    nb.dev = dev;
    nb.bytes = j4q::split_layout(r.qtype, r.rows, r.cols).total;
    *out = register_buf(nb);
    return J4Q_OK;
}

int j4q_upload_f32(const float *data, int32_t rank, const int64_t *dims, j4q_buffer *out) {
    return upload_dense(J4Q_KIND_F32, 4, data, rank, dims, out);
}

int j4q_upload_bf16(const uint16_t *data, int32_t rank, const int64_t *dims, j4q_buffer *out) {
    return upload_dense(J4Q_KIND_BF16, 2, data, rank, dims, out);
}

int j4q_download_f32(j4q_buffer h, float *out, int64_t count) {
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *b;
    int rc;
    if ((rc = get_buf(h, J4Q_KIND_F32, "download", &b))) return rc;
    if (count != elements_of(*b))
        return fail(J4Q_EINVAL, "download: buffer holds %lld floats, asked for %lld", (long long)elements_of(*b), (long long)count);
    if (count && !out) return fail(J4Q_EINVAL, "download: out is NULL");
    if ((rc = ensure_ready())) return rc;
    if (count) HIP_TRY("hipMemcpyAsync", hipMemcpyAsync(out, b->dev, (size_t)count * 4, hipMemcpyDeviceToHost, g_stream));
    HIP_TRY("hipStreamSynchronize", hipStreamSynchronize(g_stream));
    return J4Q_OK;
}

int j4q_download_bytes(j4q_buffer h, void *out, uint64_t nbytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *b;
    int rc;
    if ((rc = get_buf(h, 0, "download_bytes", &b))) return rc;
    if (b->kind == J4Q_KIND_QUANT) return fail(J4Q_EHANDLE, "download_bytes: quantized buffers are read with j4q_export_quantized");
    if (nbytes != b->bytes) return fail(J4Q_EINVAL, "download_bytes: buffer holds %llu bytes, asked for %llu", (unsigned long long)b->bytes, (unsigned long long)nbytes);
    if (nbytes && !out) return fail(J4Q_EINVAL, "download_bytes: out is NULL");
    if ((rc = ensure_ready())) return rc;
    if (nbytes) HIP_TRY("hipMemcpyAsync", hipMemcpyAsync(out, b->dev, nbytes, hipMemcpyDeviceToHost, g_stream));
    HIP_TRY("hipStreamSynchronize", hipStreamSynchronize(g_stream));
    return J4Q_OK;
}

int j4q_buffer_info(j4q_buffer h, j4q_buffer_desc *out) {
    if (!out) return fail(J4Q_EINVAL, "buffer_info: out is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *b;
    int rc;
    if ((rc = get_buf(h, 0, "buffer_info", &b))) return rc;
    memset(out, 0, sizeof *out);
    out->kind = b->kind;
    out->quant_type = b->qtype;
    out->rank = b->rank;
    out->dims[0] = b->dims[0];
    out->dims[1] = b->dims[1];
    out->bytes = b->bytes;
    out->device_ptr = b->dev;
    return J4Q_OK;
}

int j4q_buffer_stats(int64_t *live, uint64_t *bytes) {
    if (!live || !bytes) return fail(J4Q_EINVAL, "buffer_stats: NULL argument");
    std::lock_guard<std::mutex> lk(g_mu);
    int64_t n = 0;
    uint64_t b = 0;
    for (const Buf &x : g_bufs)
        if (x.live) {
            n++;
            b += x.bytes;
        }
    *live = n;
    *bytes = b;
    return J4Q_OK;
}

int j4q_release(j4q_buffer h) {
    if (h == 0) return J4Q_OK;
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *b;
    int rc;
    if ((rc = get_buf(h, 0, "release", &b))) return rc;
    if (b->pins > 0)
        return fail(J4Q_EINVAL,
                    "release: buffer 0x%llx is read by %d live decode plan(s), e.g. 0x%llx; destroy the plan first",
                    (unsigned long long)h, (int)b->pins, (unsigned long long)b->last_plan);
    if (b->dev) {
        if ((rc = ensure_ready())) return rc;
        // hipFree waits for work that may still read the buffer.
        HIP_TRY("hipFree", hipFree(b->dev));
    }
    b->dev = nullptr;
    b->live = false;
    g_free.push_back((uint32_t)((h & 0xffffffffu) - 1));
    return J4Q_OK;
}

int j4q_quant_matvec(j4q_buffer w, j4q_buffer x, j4q_buffer *y) { return matvec_common(w, x, 0, y, "quantMatvec"); }

int j4q_quant_matvec_add(j4q_buffer w, j4q_buffer x, j4q_buffer add, j4q_buffer *y) {
    if (add == 0) return fail(J4Q_EINVAL, "quantMatvecAdd: add is NULL");
    return matvec_common(w, x, add, y, "quantMatvecAdd");
}

int j4q_set_gemv_policy(int policy, int *previous) {
    if (policy != J4Q_GEMV_MATRIX_CORES && policy != J4Q_GEMV_FP32)
        return fail(J4Q_EINVAL, "set_gemv_policy: unknown policy %d (J4Q_GEMV_MATRIX_CORES or J4Q_GEMV_FP32)", policy);
    std::lock_guard<std::mutex> lk(g_mu);
    if (previous) *previous = j4q::gemv_policy();
    j4q::gemv_set_policy(policy);
    return J4Q_OK;
}

int j4q_quant_gather_row(j4q_buffer wh, int64_t row, j4q_buffer *out) {
    if (!out) return fail(J4Q_EINVAL, "quantGatherRow: out is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "quantGatherRow", &w))) return rc;
    if (row < 0 || row >= w->dims[0])
        return fail(J4Q_EINVAL, "quantGatherRow: row %lld out of range [0, %lld)", (long long)row, (long long)w->dims[0]);
    if ((rc = ensure_ready())) return rc;
    const j4q::QMat m = qmat_of(*w);
    const int qt = w->qtype;
    const int64_t K = w->dims[1];
    void *ydev;
    if ((rc = alloc_buf(J4Q_KIND_F32, 1, K, 0, (uint64_t)K * 4, out, &ydev))) return rc;
    LAUNCH_INTO("quantGatherRow", out, j4q::launch_dequant_rows(qt, m, row, 1, (float *)ydev, g_stream));
    return J4Q_OK;
}

int j4q_quant_dequantize(j4q_buffer wh, j4q_buffer *out) {
    if (!out) return fail(J4Q_EINVAL, "dequantize: out is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "dequantize", &w))) return rc;
    if ((rc = ensure_ready())) return rc;
    const j4q::QMat m = qmat_of(*w);
    const int qt = w->qtype;
    const int64_t N = w->dims[0], K = w->dims[1];
    void *ydev;
    if ((rc = alloc_buf(J4Q_KIND_F32, 2, N, K, (uint64_t)(N * K) * 4, out, &ydev))) return rc;
    LAUNCH_INTO("dequantize", out, j4q::launch_dequant_rows(qt, m, 0, N, (float *)ydev, g_stream));
    return J4Q_OK;
}

int j4q_quantize_act(j4q_buffer xh, j4q_buffer *xq, j4q_buffer *xs) {
    if (!xq || !xs) return fail(J4Q_EINVAL, "quantize_act: NULL out");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *x;
    int rc;
    if ((rc = get_buf(xh, J4Q_KIND_BF16, "quantize_act", &x))) return rc;
    if (x->rank != 2 || x->dims[0] <= 0 || x->dims[1] <= 0 || x->dims[1] % 32 != 0)
        return fail(J4Q_EINVAL, "quantize_act: x must be [M, K] with K %% 32 == 0");
    if ((rc = ensure_ready())) return rc;
    const int64_t M = x->dims[0], K = x->dims[1];
    const void *xdev = x->dev;
    void *qdev, *sdev;
    if ((rc = alloc_buf(J4Q_KIND_I8, 2, M, K, (uint64_t)(M * K), xq, &qdev))) return rc;
    if ((rc = alloc_buf(J4Q_KIND_F32, 2, M, K / 32, (uint64_t)(M * (K / 32)) * 4, xs, &sdev))) {
        drop_buf(xq);
        return rc;
    }
    const hipError_t e = j4q::launch_quantize_act((const uint16_t *)xdev, M, K, (int8_t *)qdev, (float *)sdev, g_stream);
    if (e != hipSuccess) {
        drop_buf(xq);
        drop_buf(xs);
        return hip_fail("quantize_act", e);
    }
    return J4Q_OK;
}

int j4q_quant_matmul(j4q_buffer wh, j4q_buffer xh, int variant, j4q_buffer *out) {
    if (!out) return fail(J4Q_EINVAL, "quantMatmul: out is NULL");
    if (variant != J4Q_GEMM_INT8 && variant != J4Q_GEMM_BF16) return fail(J4Q_EUNSUPPORTED, "quantMatmul: unknown variant %d", variant);
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w, *x;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "quantMatmul", &w))) return rc;
    if ((rc = get_buf(xh, J4Q_KIND_BF16, "quantMatmul", &x))) return rc;
    if ((rc = check_gemm_weights(*w, variant, "quantMatmul"))) return rc;
    if (x->rank != 2 || x->dims[1] != w->dims[1] || x->dims[0] <= 0)
        return fail(J4Q_EINVAL, "quantMatmul shape mismatch: [%lld, %lld] x [%lld, %lld]", (long long)w->dims[0],
                    (long long)w->dims[1], (long long)x->dims[0], (long long)(x->rank == 2 ? x->dims[1] : 0));
    if ((rc = check_gemm_size(x->dims[0], w->dims[1], variant, "quantMatmul"))) return rc;
    if ((rc = ensure_ready())) return rc;
    const int64_t M = x->dims[0], N = w->dims[0], K = w->dims[1];
    const j4q::QMat m = qmat_of(*w);
    const int qt = w->qtype;
    const uint16_t *xdev = (const uint16_t *)x->dev;
    // w and x are not used past this point: registering y below may move the buffer table
    void *ydev;
    if ((rc = alloc_buf(J4Q_KIND_F32, 2, M, N, (uint64_t)(M * N) * 4, out, &ydev))) return rc;
    if (variant == J4Q_GEMM_BF16) {
        void *ws = nullptr;
        const uint64_t wsb = gemm_bf16_workspace(qt, m, M);
        if (wsb) LAUNCH_INTO("hipMallocAsync", out, hipMallocAsync(&ws, wsb, g_stream));
        const hipError_t e = launch_gemm_bf16(qt, m, xdev, (float *)ydev, M, (float *)ws, g_stream);
        if (ws) (void)hipFreeAsync(ws, g_stream);
        LAUNCH_INTO("quantMatmul", out, e);
        return J4Q_OK;
    }
    void *ws = nullptr;
    const uint64_t qbytes = (uint64_t)(M * K), sbytes = (uint64_t)(M * (K / 32)) * 4;
    LAUNCH_INTO("hipMallocAsync", out, hipMallocAsync(&ws, j4q::align256(qbytes) + sbytes, g_stream));
    int8_t *xq = (int8_t *)ws;
    float *xs = (float *)((uint8_t *)ws + j4q::align256(qbytes));
    hipError_t e = j4q::launch_quantize_act(xdev, M, K, xq, xs, g_stream);
    if (e == hipSuccess) e = j4q::launch_gemm_q8_int8(m, xq, xs, (float *)ydev, M, g_stream);
    (void)hipFreeAsync(ws, g_stream);
    LAUNCH_INTO("quantMatmul", out, e);
    return J4Q_OK;
}

int j4q_quant_matvec_into(j4q_buffer wh, const float *x, const float *add, float *y, int64_t batch, void *stream) {
    if (!x || !y) return fail(J4Q_EINVAL, "quantMatvec_into: NULL x or y");
    if (!aligned(x, 16) || !aligned(y, 4) || (add && !aligned(add, 4)))
        return fail(J4Q_EINVAL, "quantMatvec_into: x must be 16-byte aligned, y and add 4-byte aligned");
    if (batch <= 0 || batch > 65535) return fail(J4Q_EINVAL, "quantMatvec_into: batch %lld out of range", (long long)batch);
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "quantMatvec_into", &w))) return rc;
    const int64_t N = w->dims[0], K = w->dims[1];
    const j4q::QMat m = qmat_of(*w);
    if (add && add != y && add < y + batch * N && y < add + batch * N)
        return fail(J4Q_EUNSUPPORTED, "quantMatvec_into: add overlaps y without being y itself");
    if (add == y && !j4q::gemv_in_place_ok(w->qtype, m, batch))
        return fail(J4Q_EUNSUPPORTED,
                    "quantMatvec_into: an add that overlaps y needs cols <= %lld (one column window) or batch >= 3 on "
                    "Q4_0/Q8_0/Q4_K/Q6_K, got cols %lld, batch %lld",
                    (long long)j4q::gemv_single_pass_cols(), (long long)K, (long long)batch);
    if ((rc = ensure_ready())) return rc;
    const hipStream_t s = pick_stream(stream);
    // partial sums of several column windows live in stream-ordered memory of the call's stream
    j4q::Workspace ws;
    const uint64_t wsb = j4q::gemv_workspace_bytes(w->qtype, m, batch);
    if (wsb) {
        void *p = nullptr;
        HIP_TRY("hipMallocAsync", hipMallocAsync(&p, wsb, s));
        ws.ptr = (float *)p;
        ws.bytes = wsb;
    }
    const hipError_t e = j4q::launch_gemv(w->qtype, m, x, add, y, batch, s, ws);
    if (ws.ptr) (void)hipFreeAsync(ws.ptr, s);
    HIP_TRY("quantMatvec_into", e);
    return J4Q_OK;
}

int j4q_quant_matmul_into(j4q_buffer wh, const uint16_t *x, int64_t m, int variant, int8_t *xq, float *xs, float *y,
                          void *stream) {
    if (!x || !y) return fail(J4Q_EINVAL, "quantMatmul_into: NULL x or y");
    if (variant != J4Q_GEMM_INT8 && variant != J4Q_GEMM_BF16) return fail(J4Q_EUNSUPPORTED, "quantMatmul_into: unknown variant %d", variant);
    if (variant == J4Q_GEMM_INT8 && (!xq || !xs)) return fail(J4Q_EINVAL, "quantMatmul_into: int8 variant needs xq and xs");
    if (!aligned(x, 16) || !aligned(y, 16) || (xq && !aligned(xq, 16)) || (xs && !aligned(xs, 16)))
        return fail(J4Q_EINVAL, "quantMatmul_into: pointers must be 16-byte aligned");
    if (m <= 0) return fail(J4Q_EINVAL, "quantMatmul_into: m must be positive");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "quantMatmul_into", &w))) return rc;
    if ((rc = check_gemm_weights(*w, variant, "quantMatmul_into"))) return rc;
    if ((rc = check_gemm_size(m, w->dims[1], variant, "quantMatmul_into"))) return rc;
    if ((rc = ensure_ready())) return rc;
    const hipStream_t s = pick_stream(stream);
    const j4q::QMat mm = qmat_of(*w);
    if (variant == J4Q_GEMM_BF16) {
        void *ws = nullptr;
        const uint64_t wsb = gemm_bf16_workspace(w->qtype, mm, m);
        if (wsb) HIP_TRY("hipMallocAsync", hipMallocAsync(&ws, wsb, s));
        const hipError_t e = launch_gemm_bf16(w->qtype, mm, x, y, m, (float *)ws, s);
        if (ws) (void)hipFreeAsync(ws, s);
        HIP_TRY("quantMatmul_into", e);
        return J4Q_OK;
    }
    HIP_TRY("quantMatmul_into", j4q::launch_quantize_act(x, m, mm.cols, xq, xs, s));
    HIP_TRY("quantMatmul_into", j4q::launch_gemm_q8_int8(mm, xq, xs, y, m, s));
    return J4Q_OK;
}

int j4q_quant_matmul_q8_into(j4q_buffer wh, const int8_t *xq, const float *xs, int64_t m, float *y, void *stream) {
    if (!xq || !xs || !y) return fail(J4Q_EINVAL, "quantMatmul_q8_into: NULL xq, xs or y");
    if (!aligned(xq, 16) || !aligned(xs, 16) || !aligned(y, 16))
        return fail(J4Q_EINVAL, "quantMatmul_q8_into: pointers must be 16-byte aligned");
    if (m <= 0) return fail(J4Q_EINVAL, "quantMatmul_q8_into: m must be positive");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "quantMatmul_q8_into", &w))) return rc;
    if ((rc = check_gemm_weights(*w, J4Q_GEMM_INT8, "quantMatmul_q8_into"))) return rc;
    if ((rc = check_gemm_size(m, w->dims[1], J4Q_GEMM_INT8, "quantMatmul_q8_into"))) return rc;
    if ((rc = ensure_ready())) return rc;
    HIP_TRY("quantMatmul_q8_into", j4q::launch_gemm_q8_int8(qmat_of(*w), xq, xs, y, m, pick_stream(stream)));
    return J4Q_OK;
}

int j4q_quant_matmul_noalloc(j4q_buffer wh, const uint16_t *x, int64_t m, int variant, float *y, void *stream) {
    if (!x || !y) return fail(J4Q_EINVAL, "quantMatmul_noalloc: NULL x or y");
    if (variant != J4Q_GEMM_INT8 && variant != J4Q_GEMM_BF16)
        return fail(J4Q_EUNSUPPORTED, "quantMatmul_noalloc: unknown variant %d", variant);
    if (!aligned(x, 16) || !aligned(y, 16)) return fail(J4Q_EINVAL, "quantMatmul_noalloc: pointers must be 16-byte aligned");
    if (m <= 0) return fail(J4Q_EINVAL, "quantMatmul_noalloc: m must be positive");
    std::lock_guard<std::mutex> lk(g_mu);
    Buf *w;
    int rc;
    if ((rc = get_buf(wh, J4Q_KIND_QUANT, "quantMatmul_noalloc", &w))) return rc;
    if ((rc = check_gemm_weights(*w, variant, "quantMatmul_noalloc"))) return rc;
    const int64_t K = w->dims[1];
    if ((rc = check_gemm_size(m, K, variant, "quantMatmul_noalloc"))) return rc;
    if (variant == J4Q_GEMM_INT8 && (uint64_t)m * (uint64_t)K > kScratchQBytes)
        return fail(J4Q_EUNSUPPORTED,
                    "quantMatmul_noalloc: the int8 variant's workspace holds m * cols <= %llu values, got %lld x %lld",
                    (unsigned long long)kScratchQBytes, (long long)m, (long long)K);
    if ((rc = ensure_ready())) return rc;
    const hipStream_t s = pick_stream(stream);
    const j4q::QMat mm = qmat_of(*w);
    if (variant == J4Q_GEMM_BF16) {
        // the K-quant kernels' split partials (at most 32 MiB) go to the engine's array
        static_assert(kScratchBytes >= (32ull << 20), "scratch holds the bf16 GEMM's workspace");
        HIP_TRY("quantMatmul_noalloc", launch_gemm_bf16(w->qtype, mm, x, y, m, (float *)g_scratch, s));
        return J4Q_OK;
    }
    int8_t *xq = (int8_t *)g_scratch;
    float *xs = (float *)((uint8_t *)g_scratch + kScratchQBytes);
    HIP_TRY("quantMatmul_noalloc", j4q::launch_quantize_act(x, m, K, xq, xs, s));
    HIP_TRY("quantMatmul_noalloc", j4q::launch_gemm_q8_int8(mm, xq, xs, y, m, s));
    return J4Q_OK;
}

int j4q_synth_quant_host(int qt, uint64_t seed, int64_t rows, int64_t cols, void *out, uint64_t nbytes) {
    Geometry g;
    int rc = check_quant_args(qt, nbytes, rows, cols, &g);
    if (rc) return rc;
    if (!out) return fail(J4Q_EINVAL, "synth_quant_host: out is NULL");
    const int64_t nb = rows * (cols / g.block_elements);
    uint8_t *o = (uint8_t *)out;
    for (int64_t bi = 0; bi < nb; bi++) j4q_synth::synth_block(qt, seed, (uint64_t)bi, cols, o + bi * g.block_bytes);
    return J4Q_OK;
}

int j4q_synth_quant_device(int qt, uint64_t seed, int64_t rows, int64_t cols, void *dout, uint64_t nbytes, void *stream) {
    Geometry g;
    int rc = check_quant_args(qt, nbytes, rows, cols, &g);
    if (rc) return rc;
    if (!dout) return fail(J4Q_EINVAL, "synth_quant_device: out is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    if ((rc = ensure_ready())) return rc;
    HIP_TRY("synth_quant_device", j4q::launch_synth_quant(qt, seed, rows, cols, (uint8_t *)dout, pick_stream(stream)));
    return J4Q_OK;
}

int j4q_synth_f32_host(uint64_t seed, int64_t n, float *out) {
    if (n < 0 || (n && !out)) return fail(J4Q_EINVAL, "synth_f32_host: bad arguments");
    for (int64_t i = 0; i < n; i++) out[i] = j4q_synth::synth_x(seed, (uint64_t)i);
    return J4Q_OK;
}

int j4q_synth_bf16_host(uint64_t seed, int64_t n, uint16_t *out) {
    if (n < 0 || (n && !out)) return fail(J4Q_EINVAL, "synth_bf16_host: bad arguments");
    for (int64_t i = 0; i < n; i++) out[i] = j4q_synth::f32_to_bf16(j4q_synth::synth_x(seed, (uint64_t)i));
    return J4Q_OK;
}

int j4q_synth_f32_device(uint64_t seed, int64_t n, float *dout, void *stream) {
    if (n < 0 || (n && !dout)) return fail(J4Q_EINVAL, "synth_f32_device: bad arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    HIP_TRY("synth_f32_device", j4q::launch_synth_f32(seed, n, dout, pick_stream(stream)));
    return J4Q_OK;
}

int j4q_synth_bf16_device(uint64_t seed, int64_t n, uint16_t *dout, void *stream) {
    if (n < 0 || (n && !dout)) return fail(J4Q_EINVAL, "synth_bf16_device: bad arguments");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    HIP_TRY("synth_bf16_device", j4q::launch_synth_bf16(seed, n, dout, pick_stream(stream)));
    return J4Q_OK;
}

int j4q_spin(uint32_t microseconds, void *stream) {
    if (microseconds > 10u * 1000u * 1000u) return fail(J4Q_EINVAL, "spin: at most 10 s");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    int khz = 0;
    HIP_TRY("hipDeviceGetAttribute", hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, g_dev));
    HIP_TRY("spin", j4q::launch_spin(microseconds, khz, pick_stream(stream)));
    return J4Q_OK;
}

int j4q_stream_read(const void *src, uint64_t nbytes, uint32_t *sink, int32_t workgroups_per_cu, int32_t loads_in_flight,
                    void *stream) {
    if (!src || !sink) return fail(J4Q_EINVAL, "stream_read: NULL pointer");
    if (loads_in_flight != 4 && loads_in_flight != 8)
        return fail(J4Q_EINVAL, "stream_read: loads_in_flight %d is not 4 or 8", loads_in_flight);
    if (nbytes % 16 != 0 || !aligned(src, 16) || nbytes >= 0x80000000ull)
        return fail(J4Q_EINVAL, "stream_read: nbytes must be a multiple of 16 below 2 GiB, src 16-byte aligned");
    if (workgroups_per_cu < 1 || workgroups_per_cu > 4) return fail(J4Q_EINVAL, "stream_read: workgroups_per_cu %d out of range [1, 4]", workgroups_per_cu);
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    hipDeviceProp_t p;
    HIP_TRY("hipGetDeviceProperties", hipGetDeviceProperties(&p, g_dev));
    HIP_TRY("stream_read", j4q::launch_stream_read(src, nbytes, sink, workgroups_per_cu * p.multiProcessorCount,
                                                   loads_in_flight, pick_stream(stream)));
    return J4Q_OK;
}

int j4q_gemv_trace(uint64_t *device_words, int64_t n_words) {
    if (device_words && (n_words < 4 || !aligned(device_words, 8)))
        return fail(J4Q_EINVAL, "gemv_trace: need at least 4 words (one wave), 8-byte aligned");
    std::lock_guard<std::mutex> lk(g_mu);
    j4q::gemv_set_trace(device_words, device_words ? n_words : 0);
    return J4Q_OK;
}

int j4q_copy(void *dst, const void *src, uint64_t nbytes, void *stream) {
    if (!dst || !src) return fail(J4Q_EINVAL, "copy: NULL pointer");
    if (nbytes % 16 != 0 || !aligned(dst, 16) || !aligned(src, 16))
        return fail(J4Q_EINVAL, "copy: nbytes must be a multiple of 16 and both pointers 16-byte aligned");
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_ready();
    if (rc) return rc;
    HIP_TRY("copy", j4q::launch_copy(dst, src, nbytes, pick_stream(stream)));
    return J4Q_OK;
}

}  // extern "C"

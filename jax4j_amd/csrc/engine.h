// Engine internals shared by the translation units behind the C ABI (api.hip owns the buffer
// table, the engine stream and the lock; gguf.hip and plan.hip use them through these calls).
#pragma once

#include <mutex>

#include "j4q_common.h"
#include "jax4j_mi355x.h"

namespace j4q {

// Sets the calling thread's j4q_last_error() message and returns `code`.
int report_error(int code, const char *fmt, ...);
// "<op> failed: <hip message> (code N)" with J4Q_ENOMEM or J4Q_EHIP.
int report_hip(const char *op, hipError_t e);

namespace abi {

// The engine lock: every entry point holds it while it reads the buffer table or launches.
std::mutex &lock();
// With the lock held: J4Q_OK once j4q_init succeeded (and the device is current).
int ready_locked();
// The engine stream (valid after ready_locked()).
hipStream_t stream();

// A resident quantized matrix, as the kernels see it.
struct QuantRef {
    int qtype;
    int64_t rows, cols;
    QMat m;
    uint64_t gguf_bytes;  // bytes of its GGUF blocks (what a GEMV streams)
};
// With the lock held: the quantized buffer behind `h`, or a J4Q_EHANDLE error naming `op`.
int quant_locked(j4q_buffer h, const char *op, QuantRef *out);
// With the lock held: records that live decode plan `plan` reads the memory of buffer `h`
// (j4q_release refuses it until unpinned), and undoes one such record.
int pin_locked(j4q_buffer h, uint64_t plan);
void unpin_locked(j4q_buffer h);
// With the lock held: a new device allocation holding the rows of `parts` in order (same
// type and column count), in the split layout; the caller owns *dev (hipFree). Synchronises.
int concat_locked(const j4q_buffer *parts, int count, void **dev, QuantRef *out);

}  // namespace abi
}  // namespace j4q

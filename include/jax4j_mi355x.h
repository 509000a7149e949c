/*
 * jax4j_mi355x.h -- C ABI of the MI355X (gfx950) GGUF quantized-matmul engine.
 *
 * This is the boundary a jax4j tensor backend binds with Java FFM downcalls: plain C types,
 * status-int returns, opaque 64-bit buffer handles and out-parameters, no C++ or torch
 * types. Every entry point names the reference interface it serves. Citations are relative
 * to the jax4j 0.2.1 checkout with these prefixes:
 *   spi/  = jax4j-core/src/main/java/com/nablatensor/jax4j/tensor/spi/
 *   core/ = jax4j-core/src/main/java/com/nablatensor/jax4j/
 *   rocm/ = jax4j-engine-rocm/src/main/java/com/nablatensor/jax4j/backend/rocm/
 *
 * Conventions
 *  - Every function returns J4Q_OK (0) or a J4Q_E* code; on failure j4q_last_error() holds a
 *    message for the calling thread. The codes map to the reference's exception types:
 *      J4Q_EINVAL, J4Q_EUNSUPPORTED, J4Q_EHANDLE -> IllegalArgumentException
 *          (core/backend/cpu/CpuBackend.java:698-701, 712-714, 757-761)
 *      J4Q_ENODEV                  -> IllegalStateException (core/tensor/BackendRegistry.java:72)
 *      J4Q_EHIP, J4Q_ENOMEM        -> RuntimeException("<op> failed: <hip message> (code N)")
 *                                      (rocm/HipRuntime.java:129-141)
 *  - Arguments are validated on the host before any HIP call, so every error path above is
 *    reachable without a GPU.
 *  - All calls are thread-safe (one engine mutex); kernels run in order on one engine stream.
 *    Functions taking a `stream` argument instead enqueue on the caller's hipStream_t
 *    (NULL = the engine stream) and return without synchronising.
 *  - Buffers returned through a j4q_buffer* are owned by the engine until j4q_release.
 */
#ifndef JAX4J_MI355X_H
#define JAX4J_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define J4Q_ABI_VERSION 1

enum j4q_status {
    J4Q_OK = 0,
    J4Q_EINVAL = 1,      /* bad shape, size, index or argument */
    J4Q_EUNSUPPORTED = 2, /* quant type or variant this engine does not implement */
    J4Q_ENODEV = 3,      /* no usable gfx950 device, or j4q_init not called successfully */
    J4Q_EHIP = 4,        /* a HIP runtime call failed */
    J4Q_ENOMEM = 5,      /* device or host allocation failed */
    J4Q_EHANDLE = 6      /* unknown, released or wrong-kind buffer handle */
};

/* GGUF type ids, identical to core/tensor/QuantType.java:5-13. */
enum j4q_quant_type { J4Q_Q4_0 = 2, J4Q_Q8_0 = 8, J4Q_Q4_K = 12, J4Q_Q6_K = 14, J4Q_Q2_0 = 42 };

/* Buffer kinds reported by j4q_buffer_info. */
enum j4q_kind { J4Q_KIND_QUANT = 1, J4Q_KIND_F32 = 2, J4Q_KIND_BF16 = 3, J4Q_KIND_I8 = 4 };

/* Prefill GEMM variants (engine-local; the SPI has no matmul over quantized weights). */
enum j4q_gemm_variant { J4Q_GEMM_INT8 = 0, J4Q_GEMM_BF16 = 1 };
/* Arithmetic of batched GEMV (j4q_set_gemv_policy). */
enum j4q_gemv_policy { J4Q_GEMV_MATRIX_CORES = 0, J4Q_GEMV_FP32 = 1 };

typedef uint64_t j4q_buffer; /* 0 is never a valid handle */

typedef struct j4q_device_props {
    char name[256];
    char arch[64];          /* e.g. "gfx950:sramecc+:xnack-" */
    int32_t device;
    int32_t compute_units;
    int32_t max_clock_khz;
    int32_t l2_bytes;
    uint64_t hbm_bytes;
} j4q_device_props;

typedef struct j4q_buffer_desc {
    int32_t kind;           /* j4q_kind */
    int32_t quant_type;     /* GGUF id for J4Q_KIND_QUANT, else 0 */
    int32_t rank;           /* 1 or 2 */
    int32_t reserved;
    int64_t dims[2];        /* logical shape; quantized: [rows, cols] as in uploadQuantized */
    uint64_t bytes;         /* device bytes holding the data */
    void *device_ptr;       /* base of the device allocation */
} j4q_buffer_desc;

/* ---- lifecycle (rocm/HipRuntime.java:145-228; rocm/RocmBackend.java:433-461) ---------- */

/* ABI version of the loaded library (J4Q_ABI_VERSION). Never fails. */
int j4q_abi_version(void);
/* 1 if a gfx950 device is present and usable, else 0. Never fails, never throws
 * (ComputeBackend.isAvailable, spi/ComputeBackend.java:43; pattern rocm/HipRuntime.java:145-158). */
int j4q_probe(void);
/* Selects `device`, creates the engine stream. Idempotent for the same device. */
int j4q_init(int device);
/* Message of the last failing call on this thread ("" if none). Never NULL. */
const char *j4q_last_error(void);
int j4q_device_info(j4q_device_props *out);
/* Block until all work queued on the engine stream is done (spi/ComputeBackend.java:277). */
int j4q_sync(void);
/* The engine stream as a hipStream_t, for callers that order their own work after it. */
int j4q_stream(void **out_stream);

/* ---- quant type table (core/tensor/QuantType.java:4-53) -------------------------------- */

/* Block geometry of a GGUF id this engine knows (QuantType rows 5-13). */
int j4q_quant_type_info(int quant_type, int32_t *block_elements, int32_t *block_bytes);
/* QuantType.byteSizeFor (QuantType.java:46-53): J4Q_EINVAL if not block-aligned. */
int j4q_quant_byte_size(int quant_type, int64_t elements, uint64_t *out_bytes);
/* QuantizedOps.supportedQuantTypes (spi/QuantizedOps.java:21; CPU set at
 * core/backend/cpu/CpuBackend.java:691-693). Writes up to `capacity` ids, sets *count. */
int j4q_supported_quant_types(int32_t *ids, int32_t capacity, int32_t *count);

/* ---- buffers (spi/ComputeBackend.java:48, 87, 280; spi/DeviceBuffer.java:26-33) -------- */

/* QuantizedOps.uploadQuantized (spi/QuantizedOps.java:24; CPU copy at CpuBackend.java:696-705).
 * Copies `nbytes` of GGUF blocks for a [rows, cols] matrix into HBM and repacks them once
 * into the engine's split layout. Requires cols % blockElements == 0 and
 * nbytes == rows * cols / blockElements * blockBytes. The caller keeps its memory. */
int j4q_upload_quantized(int quant_type, const void *blocks, uint64_t nbytes, int64_t rows, int64_t cols,
                         j4q_buffer *out);
/* Same, for a GGUF blob already resident in device memory (e.g. a file copied to HBM). */
int j4q_upload_quantized_device(int quant_type, const void *device_blocks, uint64_t nbytes, int64_t rows,
                                int64_t cols, j4q_buffer *out);
/* Writes the matrix back as GGUF blocks (bit-exact inverse of the repack). */
int j4q_export_quantized(j4q_buffer weights, void *blocks, uint64_t nbytes);
/* One matrix whose rows are the rows of `parts` in order (same quant type and column count;
 * engine-local, no SPI counterpart). Matrices that share their input, such as the q/k/v or
 * gate/up projections of a decoder layer, then run as one GEMV launch: y holds the parts'
 * outputs one after another. The parts stay valid and owned by the caller. */
int j4q_concat_rows(const j4q_buffer *parts, int32_t count, j4q_buffer *out);
/* ComputeBackend.upload for F32 data (spi/ComputeBackend.java:48). rank 1 or 2. */
int j4q_upload_f32(const float *data, int32_t rank, const int64_t *dims, j4q_buffer *out);
/* bf16 activations for the prefill GEMM (DType has no BF16, core/tensor/DType.java:19-21). */
int j4q_upload_bf16(const uint16_t *data, int32_t rank, const int64_t *dims, j4q_buffer *out);
/* ComputeBackend.download (spi/ComputeBackend.java:87): syncs, then copies `count` floats. */
int j4q_download_f32(j4q_buffer buffer, float *out, int64_t count);
/* Raw copy of any non-quantized buffer (int8 / bf16 / f32), syncing first. */
int j4q_download_bytes(j4q_buffer buffer, void *out, uint64_t nbytes);
int j4q_buffer_info(j4q_buffer buffer, j4q_buffer_desc *out);
/* ComputeBackend.release (spi/ComputeBackend.java:280). Releasing 0 is a no-op. A matrix
 * that a live decode plan reads (see j4q_decode_plan_create) is refused with J4Q_EINVAL and
 * stays valid, so memory a queued replay reads is never freed (the reference's frees never
 * race queued work either: rocm/HipBuffer.java:33-61, rocm/HipRuntime.java:246-262). */
int j4q_release(j4q_buffer buffer);
/* Live buffer handles and the device bytes they hold (engine-local accounting, the
 * counterpart of the reference's Cleaner-tracked HipBuffer frees, rocm/HipBuffer.java:31-81):
 * a call that fails after allocating releases what it allocated, so this stays unchanged. */
int j4q_buffer_stats(int64_t *live, uint64_t *device_bytes);

/* ---- the quantized ops (spi/QuantizedOps.java:27-33) ----------------------------------- */

/* QuantizedOps.quantMatvec (QuantizedOps.java:27; CpuBackend.java:708-725).
 * x with exactly cols elements (any rank) -> y F32 [rows]. Engine extension: x of shape
 * [B, cols] with B > 1 -> y F32 [B, rows] (row b of y is quantMatvec of row b of x).
 * Any block-aligned cols (CpuQ4Gemm.java:79-83): up to 32768 columns one launch holds x in
 * LDS; wider matrices run as column windows, each adding the previous window's sums. */
int j4q_quant_matvec(j4q_buffer weights, j4q_buffer x, j4q_buffer *y);
/* QuantizedOps.quantMatvecAdd (QuantizedOps.java:30; CpuBackend.java:728-736):
 * y = (W.x) + add, the add rounded separately. add needs at least as many elements as y. */
int j4q_quant_matvec_add(j4q_buffer weights, j4q_buffer x, j4q_buffer add, j4q_buffer *y);
/* QuantizedOps.quantGatherRow (QuantizedOps.java:33; CpuBackend.java:739-755): one row
 * dequantized to F32 [cols], bit-exact. Rows outside [0, rows) -> J4Q_EINVAL. */
int j4q_quant_gather_row(j4q_buffer weights, int64_t row, j4q_buffer *y);
/* Whole-matrix dequantization to F32 [rows, cols], bit-exact (engine-local export). */
int j4q_quant_dequantize(j4q_buffer weights, j4q_buffer *y);
/* Arithmetic of batched GEMV, x [B, cols] with B >= 3 (engine-local; the SPI's quantMatvec is
 * one row, CpuBackend.java:712, and the engine's batch is row b = quantMatvec of x[b]):
 *  J4Q_GEMV_MATRIX_CORES (default): launches of up to 16 batch rows on the matrix cores (Q8_0,
 *    Q4_0, Q4_K, Q6_K), W streamed once per launch; x enters the products as hi + lo fp16
 *    (22 significant bits under a power-of-two scale), the products are exact, and each row
 *    stays within 1e-4 of the fp64 product (within 4e-5 up to K = 40960 in the tests);
 *  J4Q_GEMV_FP32: every batch row on the batch-1 kernel (fp32 x, fp32 accumulation, no
 *    matrix cores; W streamed once per row), so row b equals quantMatvec of x[b] bit for bit.
 * Process-wide, for every call issued afterwards; a decode plan keeps the launches it
 * captured at creation. *previous (may be NULL) receives the policy it replaces. An unknown
 * policy: J4Q_EINVAL, nothing changed. */
int j4q_set_gemv_policy(int policy, int *previous);

/* ---- prefill GEMM (engine-local; no SPI counterpart, see CpuBackend.java:712) ---------- */

/* bf16 X [M, K] -> int8 per 32-element block with an fp32 scale per block:
 * s = amax/127, q = clamp(roundf(x * (1/s)), -127, 127) (ggml quantize_row_q8_0, fp32 scale). */
int j4q_quantize_act(j4q_buffer x_bf16, j4q_buffer *xq_i8, j4q_buffer *scales_f32);
/* Y F32 [M, N] = X [M, K] . W^T for a quantized W [N, K] (QuantizedOps.quantMatvec applied
 * to every row of X, QuantizedOps.java:27; CpuBackend.java:708-725). X is a bf16 buffer
 * (j4q_upload_bf16). J4Q_GEMM_INT8 (Q8_0 weights) quantizes X per 32 and runs int8 MFMA;
 * J4Q_GEMM_BF16 (Q8_0, Q4_0 with cols % 128 == 0, Q4_K, Q6_K) runs bf16 MFMA on W
 * dequantized to bf16 from LDS-staged blocks. Other types or variants: J4Q_EUNSUPPORTED. */
int j4q_quant_matmul(j4q_buffer weights, j4q_buffer x, int variant, j4q_buffer *y);

/* ---- stream-ordered entry points on caller memory (no sync) ----------------------------- */

/* quantMatvec / quantMatvecAdd into caller device memory: x_dev [batch, cols] fp32 (16-byte
 * aligned) and y_dev [batch, rows] fp32 (4-byte aligned); add_dev NULL or [batch, rows]
 * (4-byte aligned). add_dev may be y_dev
 * itself (a residual updated in place) for cols <= 32768, or at batch >= 3 on Q4_0, Q8_0,
 * Q4_K and Q6_K; other adds overlapping y return J4Q_EUNSUPPORTED (column windows chained
 * one after another would read it after rewriting y). A batched call over several column
 * windows keeps their partial sums in stream-ordered memory of `stream` (hipMallocAsync /
 * hipFreeAsync, batch x rows x windows floats); nothing else is allocated. */
int j4q_quant_matvec_into(j4q_buffer weights, const float *x_dev, const float *add_dev, float *y_dev,
                          int64_t batch, void *stream);
/* Prefill GEMM into caller memory (the weight types and variants of j4q_quant_matmul).
 * x_dev bf16 [m, cols]; y_dev fp32 [m, rows]. The int8 variant also needs xq_dev int8
 * [m, cols] and xs_dev fp32 [m, cols/32] as workspace; the bf16 variant ignores them. On
 * Q4_0, Q4_K and Q6_K weights with a small grid (few rows of X) the bf16 variant splits K
 * over workgroups and keeps the partial products in stream-ordered memory of `stream`
 * (hipMallocAsync / hipFreeAsync, at most 32 MiB); nothing else is allocated. */
int j4q_quant_matmul_into(j4q_buffer weights, const uint16_t *x_dev, int64_t m, int variant, int8_t *xq_dev,
                          float *xs_dev, float *y_dev, void *stream);
/* The int8 variant on activations already quantized (engine-local; no counterpart in the
 * reference): xq_dev int8 [m, cols] and xs_dev fp32 [m, cols/32] as j4q_quantize_act makes
 * them, and as j4q_quant_matmul_into's int8 variant leaves them in its xq/xs workspace, so
 * one X feeding several Q8_0 matrices is quantized once. Q8_0 weights only; y_dev fp32
 * [m, rows]; every pointer 16-byte aligned. Bit for bit the int8 variant's result for the
 * X those activations came from. */
int j4q_quant_matmul_q8_into(j4q_buffer weights, const int8_t *xq_dev, const float *xs_dev, int64_t m,
                             float *y_dev, void *stream);

/* The prefill GEMM for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same result as j4q_quant_matmul_into (bit for bit), but the int8 variant's
 * workspace (the quantized activations and their block scales) lives in one fixed engine
 * array of 36 MiB per GPU, so the call allocates nothing: x_dev bf16 [m, cols], y_dev fp32
 * [m, rows], both 16-byte aligned. The int8 variant needs m * cols <= 33554432 (32 MiB of
 * int8 activations, e.g. m = 8192 at cols = 4096), else J4Q_EUNSUPPORTED. The bf16 variant
 * over Q4_0, Q4_K and Q6_K keeps the partial products of its K split (at most 32 MiB) in the
 * same array. Every call on a GPU shares that GPU's workspace: calls that overlap on one GPU
 * (on different streams, or from threads that do not order them) race. */
int j4q_quant_matmul_noalloc(j4q_buffer weights, const uint16_t *x_dev, int64_t m, int variant, float *y_dev,
                             void *stream);

/* ---- decode-step plan (engine-local: QuantizedOps.quantMatvec / quantMatvecAdd,
 *      spi/QuantizedOps.java:27-30, composed over the layers of a decoder step) ---------- */
/* The quantized matmuls of an n-layer decode step, built once and replayed as one captured
 * HIP graph. Per layer, on the residual stream h [batch, d_model]:
 *     qkv[l]     = [q|k|v] . h          gate_up[l] = [gate|up] . h'
 *     h'         = o . x_o + h          h          = down . x_down + h'
 * and finally logits = head . h (each "+" a quantMatvecAdd: the add rounded on its own,
 * CpuBackend.java:728-736). x_o and x_down are the caller's activations (in a full model
 * the attention output and act(gate) * up, which this path does not compute). q|k|v and
 * gate|up run as one launch each when their parts share a quant type (the plan holds
 * row-concatenated copies, see j4q_concat_rows); otherwise as one launch per run of equal
 * types, with outputs in the same [batch][q|k|v] layout. Every layer must have the same
 * shapes; quant types may differ. The plan pins every matrix whose memory its graph reads
 * (o, down, the head, and any q/k/v or gate/up part not concatenated into a plan-owned
 * copy): j4q_release of one returns J4Q_EINVAL until j4q_decode_plan_destroy. The io
 * pointers are caller memory bound at creation (the graph records them) and must outlive
 * the plan. The GEMV trace (j4q_gemv_trace) is off inside a plan's graph. */
typedef uint64_t j4q_plan; /* 0 is never a valid handle */

typedef struct j4q_decode_layer {
    j4q_buffer q, k, v;   /* [q_rows | kv_rows | kv_rows, d_model] */
    j4q_buffer o;         /* [d_model, o_cols] */
    j4q_buffer gate, up;  /* [ffn, d_model] */
    j4q_buffer down;      /* [d_model, ffn] */
} j4q_decode_layer;

typedef struct j4q_decode_io {
    float *h;             /* [batch, d_model] residual stream, read and updated in place (16-byte aligned) */
    const float *x_o;     /* [batch, o_cols] input of every layer's o (16-byte aligned) */
    const float *x_down;  /* [batch, ffn] input of every layer's down (16-byte aligned) */
    float *qkv;           /* [layers][batch][q_rows + 2 kv_rows] */
    float *gate_up;       /* [layers][batch][2 ffn] */
    float *logits;        /* [batch, vocab]; may be NULL when there is no head */
} j4q_decode_io;

typedef struct j4q_decode_plan_desc {
    int32_t layers;
    int32_t graph;          /* 1: one step replays as one captured HIP graph */
    int64_t batch, d_model, qkv_rows, o_cols, ffn, vocab;
    int64_t gemvs_per_step; /* quantized GEMV calls per step (a fused group counts once) */
    uint64_t weight_bytes;  /* GGUF bytes of every matrix one step streams */
    uint64_t plan_bytes;    /* device memory the plan owns (fused copies, residual buffer) */
} j4q_decode_plan_desc;

/* head may be 0 (no output head). batch in [1, 65535]. */
int j4q_decode_plan_create(const j4q_decode_layer *layers, int32_t n_layers, j4q_buffer head, int64_t batch,
                           const j4q_decode_io *io, j4q_plan *out);
/* Enqueues one step on `stream` (NULL = the engine stream); does not synchronise. */
int j4q_decode_plan_run(j4q_plan plan, void *stream);
int j4q_decode_plan_info(j4q_plan plan, j4q_decode_plan_desc *out);
/* Waits for the device, then frees the graph and the plan's own buffers. 0 is a no-op. */
int j4q_decode_plan_destroy(j4q_plan plan);

/* ---- GGUF files (the step before uploadQuantized; engine-local) ---------------------- */
/* The reference receives quantized blobs from an external caller (spi/QuantizedOps.java:24)
 * and knows the GGUF type ids (core/tensor/QuantType.java:3-13); this reader supplies them
 * from a .gguf file (v2/v3). The file is mapped read-only and fully bounds-checked on open;
 * malformed files fail with J4Q_EINVAL and a message naming the byte position. */
typedef uint64_t j4q_gguf; /* 0 is never a valid handle */

typedef struct j4q_gguf_info {
    uint32_t version;
    uint32_t reserved;
    int64_t tensor_count;
    int64_t metadata_count;
    uint64_t alignment;    /* general.alignment, default 32 */
    uint64_t data_offset;  /* file offset of the tensor data section */
    uint64_t file_bytes;
} j4q_gguf_info;

typedef struct j4q_gguf_tensor {
    char name[256];
    int32_t type_id;       /* ggml type id (QuantType ids for the types the reference knows) */
    int32_t n_dims;        /* 1..4 */
    int64_t dims[4];       /* innermost first: a [rows, cols] matrix has dims {cols, rows, 1, 1} */
    uint64_t offset;       /* absolute file offset of the data */
    uint64_t nbytes;       /* 0 if the type's block geometry is unknown */
} j4q_gguf_tensor;

int j4q_gguf_open(const char *path, j4q_gguf *out);
/* Unmaps the file. Closing 0 is a no-op. */
int j4q_gguf_close(j4q_gguf f);
int j4q_gguf_file_info(j4q_gguf f, j4q_gguf_info *out);
int j4q_gguf_tensor_info(j4q_gguf f, int64_t index, j4q_gguf_tensor *out);
int j4q_gguf_find_tensor(j4q_gguf f, const char *name, int64_t *index);
/* Metadata entry `index`: key (truncated to cap - 1 bytes), GGUF value type (0 u8 .. 12 f64),
 * array element type and count (string: count = byte length). Any out pointer may be NULL. */
int j4q_gguf_meta_key(j4q_gguf f, int64_t index, char *key, int32_t cap, int32_t *type, int32_t *elem_type,
                      uint64_t *count);
/* Scalar metadata value, zero-extended into 8 bytes, and its GGUF type. */
int j4q_gguf_meta_scalar(j4q_gguf f, const char *key, int32_t *type, void *value8);
/* String metadata value (NUL-terminated, truncated to cap - 1 bytes) and its full length. */
int j4q_gguf_meta_string(j4q_gguf f, const char *key, char *out, uint64_t cap, uint64_t *length);
/* Copies tensor `index`'s blocks (exactly nbytes) to host memory. */
int j4q_gguf_read_tensor(j4q_gguf f, int64_t index, void *dst, uint64_t nbytes);
/* QuantizedOps.uploadQuantized of tensor `index` straight from the mapping (rows = product of
 * dims[1..3], cols = dims[0]); the same type and size rules as j4q_upload_quantized. */
int j4q_gguf_upload(j4q_gguf f, int64_t index, j4q_buffer *out);

/* ---- seeded synthetic inputs (benchmark support; no reference counterpart) ------------- */

/* GGUF blocks for a [rows, cols] matrix with the benchmark distributions, written to host
 * memory; bit-identical to the device generator below. */
int j4q_synth_quant_host(int quant_type, uint64_t seed, int64_t rows, int64_t cols, void *out, uint64_t nbytes);
int j4q_synth_quant_device(int quant_type, uint64_t seed, int64_t rows, int64_t cols, void *device_out,
                           uint64_t nbytes, void *stream);
/* N(0,1) fp32 values, or their round-to-nearest-even bf16. */
int j4q_synth_f32_host(uint64_t seed, int64_t n, float *out);
int j4q_synth_bf16_host(uint64_t seed, int64_t n, uint16_t *out);
int j4q_synth_f32_device(uint64_t seed, int64_t n, float *device_out, void *stream);
int j4q_synth_bf16_device(uint64_t seed, int64_t n, uint16_t *device_out, void *stream);
/* Occupies `stream` for `microseconds` (<= 10 s) of device wall-clock time, so a host can
 * queue many short launches behind it and time them back to back with events. */
int j4q_spin(uint32_t microseconds, void *stream);
/* Streaming copy of `nbytes` (a multiple of 16; both pointers 16-byte aligned) with 128-bit
 * loads and stores: a kernel of known traffic, used to scale HBM byte counters. */
int j4q_copy(void *device_dst, const void *device_src, uint64_t nbytes, void *stream);
/* Reads `nbytes` (a multiple of 16 below 2 GiB, src 16-byte aligned) once with 128-bit
 * non-temporal loads, each wave one contiguous segment, and writes nothing but, in a case no
 * input produces in practice, one word per workgroup to `sink` (workgroups_per_cu x CUs
 * words): the practical HBM read ceiling of a single launch of that size, against which the
 * GEMV launches are measured. 1..4 workgroups of 512 threads per CU; each wave keeps
 * loads_in_flight (4 or 8) 1 KB loads in flight. */
int j4q_stream_read(const void *device_src, uint64_t nbytes, uint32_t *sink, int32_t workgroups_per_cu,
                    int32_t loads_in_flight, void *stream);
/* Per-wave timeline of the batch-1 vector-ALU GEMV launches enqueued while it is set:
 * wave w < n_words / 4 writes device_words[4 w .. 4 w + 3] = {wall clock (the device's
 * constant-rate clock, hipDeviceAttributeWallClockRate) at entry, after x is staged, after
 * its last item, items | (hardware CU id << 32)}; every such launch overwrites them. NULL turns
 * it off. Decode plans capture their graphs with the trace off. */
int j4q_gemv_trace(uint64_t *device_words, int64_t n_words);

#ifdef __cplusplus
}
#endif
#endif /* JAX4J_MI355X_H */

// Decode-step plan: the quantized matmuls of an n-layer decoder step, built once and replayed
// as one captured HIP graph (engine-local; each GEMV is QuantizedOps.quantMatvec or
// quantMatvecAdd, spi/QuantizedOps.java:27-30, with the CPU semantics of
// core/backend/cpu/CpuBackend.java:708-736).
//
// Per layer, on the residual stream h [batch, d_model]:
//   qkv[l]     = [q|k|v] . h                 (one launch when q, k, v share a quant type)
//   h'         = o . x_o + h                 (quantMatvecAdd, the add rounded on its own)
//   gate_up[l] = [gate|up] . h'
//   h          = down . x_down + h'
// then logits = head . h. x_o and x_down are the caller's activations (what attention and
// the FFN activation produce in a full model; those ops are not part of this path). Every
// GEMV therefore waits for the one before it, as in a real decode step.
//
// The residual adds run out of place between h and a second buffer the plan owns, so no
// launch reads an add it has already overwritten (every K, every batch size takes the same
// kernels as the single calls); two adds per layer leave the result in h.
// Matrices of one group (q|k|v, gate|up) are concatenated by rows once, at creation, into
// copies the plan owns. Runs of parts with different quant types launch separately; with
// batch > 1 their outputs go through plan-owned scratch and a strided row copy, so the
// output layout [batch][q|k|v] never depends on the types.
#include <stdio.h>
#include <string.h>

#include <vector>

#include "engine.h"

namespace j4q {
void gemv_set_trace(uint64_t *words, int64_t n);
int64_t gemv_get_trace(uint64_t **words);

namespace {

// dst[b * dst_pitch + c] = src[b * cols + c] for b < batch, c < cols (floats).
__global__ void __launch_bounds__(256)
copy_rows_kernel(float *__restrict__ dst, int64_t dst_pitch, const float *__restrict__ src, int64_t cols, int64_t batch) {
    const int64_t n = cols * batch;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t b = i / cols, c = i - b * cols;
        dst[b * dst_pitch + c] = src[i];
    }
}

struct Op {
    bool gemv;
    // GEMV
    int qt;
    QMat m;
    const float *x, *add;
    float *y;
    // row copy
    float *dst;
    int64_t dst_pitch, cols;
    const float *src;
};

struct Plan {
    j4q_decode_plan_desc desc{};
    int64_t batch = 0;
    Workspace ws;  // partial sums of batched GEMVs over several column windows (plan-owned)
    std::vector<Op> ops;
    std::vector<void *> owned;
    // caller buffers whose memory the graph reads (o, down, the head, and group parts that were
    // not concatenated into plan-owned copies): pinned while the plan lives, so j4q_release
    // cannot free memory a replay still reads
    std::vector<j4q_buffer> reads;
    bool pinned = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uint32_t gen = 0;
    bool live = false;
};

std::vector<Plan> g_plans;

hipError_t enqueue(const Plan &p, hipStream_t s) {
    for (const Op &o : p.ops) {
        hipError_t e;
        if (o.gemv) {
            e = launch_gemv(o.qt, o.m, o.x, o.add, o.y, p.batch, s, p.ws);
        } else {
            const int64_t n = o.cols * p.batch;
            const int64_t blocks = (n + 255) / 256;
            copy_rows_kernel<<<(unsigned)(blocks < 1024 ? blocks : 1024), 256, 0, s>>>(o.dst, o.dst_pitch, o.src, o.cols,
                                                                                   p.batch);
            e = hipGetLastError();
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

void free_plan(Plan &p) {
    if (p.pinned)
        for (j4q_buffer h : p.reads) abi::unpin_locked(h);
    if (p.exec) (void)hipGraphExecDestroy(p.exec);
    if (p.graph) (void)hipGraphDestroy(p.graph);
    for (void *d : p.owned) (void)hipFree(d);
    const uint32_t gen = p.gen;
    p = Plan();
    p.gen = gen;
}

Plan *lookup(j4q_plan h) {
    const uint64_t lo = h & 0xffffffffu;
    if (lo == 0 || lo > g_plans.size()) return nullptr;
    Plan &p = g_plans[lo - 1];
    return p.live && p.gen == (uint32_t)(h >> 32) ? &p : nullptr;
}

bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// The GEMVs of one group (q|k|v or gate|up) with input x, writing [batch][group rows] at
// out: runs of consecutive parts with one quant type are concatenated into a plan-owned
// matrix; with several runs and batch > 1 each run writes scratch and is copied into place.
int build_group(Plan &p, const j4q_buffer *parts, int count, const char *what, const float *x, float *out,
                int64_t group_rows) {
    using abi::QuantRef;
    std::vector<QuantRef> refs((size_t)count);
    for (int i = 0; i < count; i++) {
        const int rc = abi::quant_locked(parts[i], what, &refs[(size_t)i]);
        if (rc) return rc;
    }
    int64_t row0 = 0;
    for (int i = 0; i < count;) {
        int j = i + 1;
        while (j < count && refs[(size_t)j].qtype == refs[(size_t)i].qtype) j++;
        QuantRef run = refs[(size_t)i];
        if (j - i > 1) {
            void *dev = nullptr;
            const int rc = abi::concat_locked(parts + i, j - i, &dev, &run);
            if (rc) return rc;
            p.owned.push_back(dev);
            p.desc.plan_bytes += split_layout(run.qtype, run.rows, run.cols).total;
        } else {
            run.gguf_bytes = refs[(size_t)i].gguf_bytes;
            p.reads.push_back(parts[i]);
        }
        Op g{};
        g.gemv = true;
        g.qt = run.qtype;
        g.m = run.m;
        g.x = x;
        if (run.rows == group_rows || p.batch == 1) {
            g.y = out + row0;
            p.ops.push_back(g);
        } else {
            void *scratch = nullptr;
            const hipError_t e = hipMalloc(&scratch, (size_t)(p.batch * run.rows) * 4);
            if (e != hipSuccess) return report_hip("decode plan scratch", e);
            p.owned.push_back(scratch);
            p.desc.plan_bytes += (uint64_t)(p.batch * run.rows) * 4;
            g.y = (float *)scratch;
            p.ops.push_back(g);
            Op c{};
            c.gemv = false;
            c.dst = out + row0;
            c.dst_pitch = group_rows;
            c.cols = run.rows;
            c.src = (const float *)scratch;
            p.ops.push_back(c);
        }
        p.desc.gemvs_per_step++;
        p.desc.weight_bytes += run.gguf_bytes;
        row0 += run.rows;
        i = j;
    }
    return J4Q_OK;
}

int one_gemv(Plan &p, j4q_buffer w, const char *what, const float *x, const float *add, float *y) {
    abi::QuantRef r;
    const int rc = abi::quant_locked(w, what, &r);
    if (rc) return rc;
    Op g{};
    g.gemv = true;
    g.qt = r.qtype;
    g.m = r.m;
    g.x = x;
    g.add = add;
    g.y = y;
    p.ops.push_back(g);
    p.reads.push_back(w);
    p.desc.gemvs_per_step++;
    p.desc.weight_bytes += r.gguf_bytes;
    return J4Q_OK;
}

// Shapes of every layer must agree, so the caller's buffers have one layout.
int check_shapes(const j4q_decode_layer *layers, int32_t n, j4q_buffer head, j4q_decode_plan_desc *d) {
    using abi::QuantRef;
    for (int32_t l = 0; l < n; l++) {
        const j4q_decode_layer &L = layers[l];
        const j4q_buffer hs[7] = {L.q, L.k, L.v, L.o, L.gate, L.up, L.down};
        static const char *names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
        QuantRef r[7];
        for (int i = 0; i < 7; i++) {
            char op[64];
            snprintf(op, sizeof op, "decode plan layer %d %s", l, names[i]);
            const int rc = abi::quant_locked(hs[i], op, &r[i]);
            if (rc) return rc;
        }
        const int64_t dm = r[0].cols, qkv = r[0].rows + r[1].rows + r[2].rows, ffn = r[4].rows;
        const bool ok = r[1].cols == dm && r[2].cols == dm && r[3].rows == dm && r[4].cols == dm && r[5].cols == dm &&
                        r[5].rows == ffn && r[6].rows == dm && r[6].cols == ffn;
        if (!ok)
            return report_error(J4Q_EINVAL,
                                "decode plan layer %d: shapes do not chain (q/k/v/gate/up need %lld columns, o and down "
                                "%lld rows, up as many rows as gate, down as many columns as gate has rows)",
                                l, (long long)dm, (long long)dm);
        if (l == 0) {
            d->d_model = dm;
            d->qkv_rows = qkv;
            d->o_cols = r[3].cols;
            d->ffn = ffn;
        } else if (dm != d->d_model || qkv != d->qkv_rows || r[3].cols != d->o_cols || ffn != d->ffn) {
            return report_error(J4Q_EINVAL, "decode plan layer %d: shapes differ from layer 0", l);
        }
    }
    d->vocab = 0;
    if (head) {
        QuantRef r;
        const int rc = abi::quant_locked(head, "decode plan head", &r);
        if (rc) return rc;
        if (r.cols != d->d_model)
            return report_error(J4Q_EINVAL, "decode plan head has %lld columns, d_model is %lld", (long long)r.cols,
                                (long long)d->d_model);
        d->vocab = r.rows;
    }
    return J4Q_OK;
}

}  // namespace
}  // namespace j4q

using namespace j4q;

extern "C" {

int j4q_decode_plan_create(const j4q_decode_layer *layers, int32_t n_layers, j4q_buffer head, int64_t batch,
                           const j4q_decode_io *io, j4q_plan *out) {
    if (!layers || !io || !out) return report_error(J4Q_EINVAL, "decode plan: NULL argument");
    if (n_layers < 1 || n_layers > 4096) return report_error(J4Q_EINVAL, "decode plan: %d layers out of range [1, 4096]", n_layers);
    if (batch < 1 || batch > 65535) return report_error(J4Q_EINVAL, "decode plan: batch %lld out of range [1, 65535]", (long long)batch);
    if (!io->h || !io->x_o || !io->x_down || !io->qkv || !io->gate_up || (head && !io->logits))
        return report_error(J4Q_EINVAL, "decode plan: a required io pointer is NULL");
    if (!aligned(io->h, 16) || !aligned(io->x_o, 16) || !aligned(io->x_down, 16) || !aligned(io->qkv, 4) ||
        !aligned(io->gate_up, 4) || (io->logits && !aligned(io->logits, 4)))
        return report_error(J4Q_EINVAL, "decode plan: h, x_o and x_down must be 16-byte aligned, outputs 4-byte aligned");
    std::lock_guard<std::mutex> lk(abi::lock());
    int rc = abi::ready_locked();
    if (rc) return rc;
    Plan p;
    p.batch = batch;
    p.desc.layers = n_layers;
    p.desc.batch = batch;
    if ((rc = check_shapes(layers, n_layers, head, &p.desc))) return rc;
    const int64_t B = batch, D = p.desc.d_model;
    void *h2 = nullptr;
    hipError_t e = hipMalloc(&h2, (size_t)(B * D) * 4);
    if (e != hipSuccess) return report_hip("decode plan residual buffer", e);
    p.owned.push_back(h2);
    p.desc.plan_bytes += (uint64_t)(B * D) * 4;
    float *h = io->h, *h_alt = (float *)h2;
    for (int32_t l = 0; l < n_layers && !rc; l++) {
        const j4q_decode_layer &L = layers[l];
        const j4q_buffer qkv[3] = {L.q, L.k, L.v}, gu[2] = {L.gate, L.up};
        float *qkv_out = io->qkv + (int64_t)l * B * p.desc.qkv_rows;
        float *gu_out = io->gate_up + (int64_t)l * B * 2 * p.desc.ffn;
        if (!rc) rc = build_group(p, qkv, 3, "decode plan q|k|v", h, qkv_out, p.desc.qkv_rows);
        if (!rc) rc = one_gemv(p, L.o, "decode plan o", io->x_o, h, h_alt);
        if (!rc) rc = build_group(p, gu, 2, "decode plan gate|up", h_alt, gu_out, 2 * p.desc.ffn);
        if (!rc) rc = one_gemv(p, L.down, "decode plan down", io->x_down, h_alt, h);
    }
    if (!rc && head) rc = one_gemv(p, head, "decode plan head", h, nullptr, io->logits);
    uint64_t wsb = 0;
    for (const Op &o : p.ops) {
        const uint64_t b = o.gemv ? gemv_workspace_bytes(o.qt, o.m, batch) : 0;
        if (b > wsb) wsb = b;
    }
    if (!rc && wsb) {
        void *d = nullptr;
        e = hipMalloc(&d, wsb);
        if (e != hipSuccess) {
            rc = report_hip("decode plan workspace", e);
        } else {
            p.owned.push_back(d);
            p.ws.ptr = (float *)d;
            p.ws.bytes = wsb;
            p.desc.plan_bytes += wsb;
        }
    }
    if (rc) {
        free_plan(p);
        return rc;
    }
    // Capture one step on a private stream (thread-local mode: other threads' HIP calls are
    // unaffected) and instantiate it; replays then cost one graph launch. The GEMV trace is
    // off while capturing: a graph that recorded the trace buffer would keep writing it after
    // the caller turned the trace off and freed it.
    uint64_t *trace_words = nullptr;
    const int64_t trace_n = gemv_get_trace(&trace_words);
    gemv_set_trace(nullptr, 0);
    hipStream_t cs = nullptr;
    e = hipStreamCreateWithFlags(&cs, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        const hipError_t le = enqueue(p, cs);
        e = hipStreamEndCapture(cs, &p.graph);
        if (le != hipSuccess) e = le;
    }
    gemv_set_trace(trace_words, trace_n);
    if (e == hipSuccess) e = hipGraphInstantiate(&p.exec, p.graph, nullptr, nullptr, 0);
    if (cs) (void)hipStreamDestroy(cs);
    if (e != hipSuccess) {
        free_plan(p);
        return report_hip("decode plan graph capture", e);
    }
    p.desc.graph = 1;
    uint32_t slot = 0;
    while (slot < g_plans.size() && g_plans[slot].live) slot++;
    if (slot == g_plans.size()) g_plans.emplace_back();
    p.gen = g_plans[slot].gen + 1;
    p.live = true;
    const j4q_plan handle = ((uint64_t)p.gen << 32) | (uint64_t)(slot + 1);
    // every handle was looked up under this same lock hold, so pinning cannot fail
    for (j4q_buffer h : p.reads) (void)abi::pin_locked(h, handle);
    p.pinned = true;
    g_plans[slot] = std::move(p);
    *out = handle;
    return J4Q_OK;
}

int j4q_decode_plan_run(j4q_plan plan, void *stream) {
    std::lock_guard<std::mutex> lk(abi::lock());
    Plan *p = lookup(plan);
    if (!p) return report_error(J4Q_EHANDLE, "decode plan run: unknown or destroyed plan 0x%llx", (unsigned long long)plan);
    int rc = abi::ready_locked();
    if (rc) return rc;
    const hipError_t e = hipGraphLaunch(p->exec, stream ? (hipStream_t)stream : abi::stream());
    if (e != hipSuccess) return report_hip("decode plan run", e);
    return J4Q_OK;
}

int j4q_decode_plan_info(j4q_plan plan, j4q_decode_plan_desc *out) {
    if (!out) return report_error(J4Q_EINVAL, "decode plan info: out is NULL");
    std::lock_guard<std::mutex> lk(abi::lock());
    Plan *p = lookup(plan);
    if (!p) return report_error(J4Q_EHANDLE, "decode plan info: unknown or destroyed plan 0x%llx", (unsigned long long)plan);
    *out = p->desc;
    return J4Q_OK;
}

int j4q_decode_plan_destroy(j4q_plan plan) {
    if (plan == 0) return J4Q_OK;
    std::lock_guard<std::mutex> lk(abi::lock());
    Plan *p = lookup(plan);
    if (!p) return report_error(J4Q_EHANDLE, "decode plan destroy: unknown or destroyed plan 0x%llx", (unsigned long long)plan);
    int rc = abi::ready_locked();
    if (rc) return rc;
    // replays may still run on any stream: wait for the device before the graph and the
    // plan's buffers go away
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return report_hip("decode plan destroy", e);
    free_plan(*p);
    return J4Q_OK;
}

}  // extern "C"

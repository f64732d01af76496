// ggml-mi355x.cpp -- the MI355X ggml backend: registry, device, buffer type,
// buffers with weight prepack at upload, and graph_compute dispatching the
// decode hot path to the gfx950 kernels through their C ABI.
//
// Reference behaviour mirrored (patch = patches/ascend310b4-llama-cpp.patch):
//   get_alloc_size   pad to 256 B + planar side copy for Q8_0/Q4_0 matmul weights
//                    (cf. ggml_cann_310b_a8w8_size / _nz_size, patch:1535-1562, 1810-1847)
//   set_tensor       ND bytes at tensor->data, side copy built when the tensor is
//                    complete; chunked and concurrent uploads through a per-tensor
//                    tracker under a mutex (patch:1647-1653, 1700-1809)
//   supports_op      MUL_MAT with M <= 8, FLASH_ATTN_EXT with one query row per sequence
//                    or up to 8 rows of one sequence
//                    (cf. patch:1925-1983), everything else false -> CPU fallback
//   graph_compute    per-node dispatch on one stream (patch:1884-1922); runtime
//                    errors abort like ACL_CHECK; GGML_MI355X_TRACE_NODE_SYNC=1
//                    synchronizes and logs after every node (patch:1887-1921)
// MI355X-specific: runs of adjacent nodes of the decode graph fuse into single
// launches (RMSNorm into the GEMV prologue; bias, residual, RoPE and the KV-cache
// write into GEMV epilogues; SwiGLU into the next GEMV's activation quantization),
// consecutive MUL_MATs sharing their activation run as one grouped GEMV launch,
// and a graph whose nodes did not change since the last call is replayed as a
// captured HIP graph.
#include "ggml-mi355x.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml_mi355x_kernels.h"

#define MI_HIP_CHECK(expr)                                                                                 \
    do {                                                                                                   \
        hipError_t e_ = (expr);                                                                            \
        if (e_ != hipSuccess) GGML_ABORT("MI355X: %s failed: %s", #expr, hipGetErrorString(e_));          \
    } while (0)

#define MI_K_CHECK(expr)                                                                                   \
    do {                                                                                                   \
        int r_ = (expr);                                                                                   \
        if (r_ != MI_OK) GGML_ABORT("MI355X: %s failed (%d): %s", #expr, r_, mi_last_error());            \
    } while (0)

namespace {

// ------------------------------------------------------------------ env flags (read once)

bool env_flag(const char *name, bool def) {
    const char *v = getenv(name);
    if (!v || !*v) return def;
    std::string s(v);
    for (auto &c : s) c = (char)tolower(c);
    return !(s == "0" || s == "off" || s == "false" || s == "no" || s == "disable");
}

bool prepack_enabled() {
    static const bool on = env_flag("GGML_MI355X_PREPACK", true);
    return on;
}
// read when a backend is created (one process may hold backends with and without replay)
bool graphs_env() { return env_flag("GGML_MI355X_GRAPHS", true) && !env_flag("GGML_MI355X_TRACE_NODE_SYNC", false); }
bool trace_node_sync() {
    static const bool on = env_flag("GGML_MI355X_TRACE_NODE_SYNC", false);
    return on;
}
// read when a backend is created, so each backend instance keeps its own setting
bool fusion_env() { return env_flag("GGML_MI355X_FUSION", true); }
int q8_rounding() {
    static const int r = [] {
        const char *v = getenv("GGML_MI355X_Q8_ROUNDING");
        return (v && strcmp(v, "ref") == 0) ? MI_Q8_ROUND_REF : MI_Q8_ROUND_X86;
    }();
    return r;
}

// ------------------------------------------------------------------ weights

// Same weight classes as the CANN backend's is_matmul_weight (aclnn_ops.h): the
// projection and output matrices of a transformer.
bool is_matmul_weight(const ggml_tensor *t) {
    static const char *suffixes[] = {"output.weight",   "attn_q.weight",   "attn_k.weight", "attn_v.weight",
                                     "attn_output.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    const size_t ln = strlen(t->name);
    for (const char *s : suffixes) {
        const size_t ls = strlen(s);
        if (ln >= ls && strcmp(t->name + ln - ls, s) == 0) return true;
    }
    return false;
}

// A8W8 from F16 weights (the reference's GGML_CANN_A8W8, patch:1472-1479): F16 projection
// weights get a Q8_0 side copy quantized at upload.  Read on every call (not cached) so a
// process can load one model with it and one without; get_alloc_size, init_tensor and
// set_tensor of one model load see the same environment.
bool a8w8_enabled() { return env_flag("GGML_MI355X_A8W8", false); }

// GGML_MI355X_A8W8_DISABLE_LAYERS="0-2,27": layers whose weights stay F16 (the reference's
// GGML_CANN_A8W8_DISABLE_LAYERS, patch:1481-1518: comma-separated layers or lo-hi ranges)
bool a8w8_layer_disabled(const char *name) {
    const char *p = strstr(name, "blk.");
    if (!p || !isdigit((unsigned char)p[4])) return false;
    const long layer = strtol(p + 4, nullptr, 10);
    const char *v = getenv("GGML_MI355X_A8W8_DISABLE_LAYERS");
    if (!v) return false;
    std::string s(v);
    size_t pos = 0;
    while (pos < s.size()) {
        size_t end = s.find(',', pos);
        if (end == std::string::npos) end = s.size();
        std::string item = s.substr(pos, end - pos);
        item.erase(std::remove(item.begin(), item.end(), ' '), item.end());
        if (!item.empty()) {
            char *dash = nullptr;
            const long lo = strtol(item.c_str(), &dash, 10);
            const long hi = (dash && *dash == '-') ? strtol(dash + 1, nullptr, 10) : lo;
            if (layer >= lo && layer <= hi) return true;
        }
        pos = end + 1;
    }
    return false;
}

// the projection classes quantized from F16: the reference's A8W8 takes the FFN matrices
// (patch:1520-1533); here every per-layer projection (q/k/v/o/gate/up/down), since the
// decode's A8W8 GEMVs serve all of them.  The tied output head stays F16.
bool is_a8w8_weight(const ggml_tensor *t) {
    return t->type == GGML_TYPE_F16 && strncmp(t->name, "blk.", 4) == 0 && is_matmul_weight(t) && a8w8_enabled() &&
           !a8w8_layer_disabled(t->name);
}

// The packed side-copy format of a weight (GGML_TYPE_COUNT: no side copy): Q8_0 and Q4_0
// matmul weights are re-laid out; F16 projection weights on the A8W8 path get Q8_0.
ggml_type side_fmt(const ggml_tensor *t) {
    if (!prepack_enabled() || t->ne[2] != 1 || t->ne[3] != 1 || t->view_src != nullptr || t->ne[0] % 32 != 0)
        return GGML_TYPE_COUNT;
    if ((t->type == GGML_TYPE_Q8_0 || t->type == GGML_TYPE_Q4_0) && is_matmul_weight(t)) return t->type;
    if (is_a8w8_weight(t)) return GGML_TYPE_Q8_0;
    return GGML_TYPE_COUNT;
}

bool prepack_eligible(const ggml_tensor *t) { return side_fmt(t) != GGML_TYPE_COUNT; }

size_t side_offset(const ggml_tensor *t) { return GGML_PAD(ggml_nbytes(t), 256); }

size_t packed_size(const ggml_tensor *t) {
    return side_fmt(t) == GGML_TYPE_Q8_0 ? mi_q8_0_packed_size(t->ne[1], t->ne[0])
                                         : mi_q4_0_packed_size(t->ne[1], t->ne[0]);
}

struct TensorExtra {
    void *packed = nullptr;  // planar side copy (device)
    ggml_type fmt = GGML_TYPE_COUNT;  // its format (Q8_0 for an F16 weight quantized at upload)
    bool ready = false;      // side copy built
    const float *inv_s = nullptr;  // SmoothQuant reciprocal factors (device), owned by the buffer
    const float *s = nullptr;      // SmoothQuant factors folded into an F16 weight's Q8_0 copy (device)
    std::mutex mtx;                // orders a side-copy build against a change of s
};

// the weight format the kernels see: the side copy's when there is one
ggml_type packed_fmt(const ggml_tensor *w) {
    const TensorExtra *ex = (const TensorExtra *)w->extra;
    return ex ? ex->fmt : w->type;
}

struct SetTracker {
    std::mutex mtx;
    size_t bytes_written = 0;
    size_t total_bytes = 0;
};

// ------------------------------------------------------------------ device / buffer type

struct DeviceCtx {
    int device = 0;
    std::string name;
    std::string description;
    ggml_backend_buffer_type buft;
    std::string buft_name;
};

struct BufferCtx {
    int device = 0;
    void *dev_ptr = nullptr;
    size_t size = 0;
    hipStream_t stream = nullptr;  // upload / prepack stream of this buffer
    std::mutex mtx;
    std::unordered_map<const ggml_tensor *, std::unique_ptr<SetTracker>> trackers;
    std::vector<std::unique_ptr<TensorExtra>> extras;
    std::vector<void *> owned;  // SmoothQuant factor copies
    std::unordered_map<std::string, void *> factors_by_content;
};

struct BackendCtx {
    int device = 0;
    bool fuse = true;
    std::string name;
    hipStream_t stream = nullptr;
    void *scratch = nullptr;
    size_t scratch_size = 0;
    void *fa_ws = nullptr;
    size_t fa_ws_size = 0;
    // per-32-block arrival counters of the A8W8 gate/up pair launch (zeroed once, left zero)
    unsigned *ffn_counters = nullptr;
    int64_t ffn_counters_words = 0;
    // the rotation table of the current graph's position (built by its first fused q/k/v
    // chain, read by every layer's)
    float *rope_tab = nullptr;  // [2][512]
    struct {
        const void *pos = nullptr;
        int64_t hd = 0;
        float freq_base = 0, freq_scale = 0, attn_factor = 0;
        bool valid = false;
    } rope_key;
    // the persistent layer-stack decode (created for the first run of layers it fuses)
    bool persist_on = false;      // GGML_MI355X_PERSIST, read when the backend is created
    std::string persist_trace;    // GGML_MI355X_PERSIST_TRACE: file for the last launch's phase timestamps
    void *persist = nullptr;
    int persist_layers = 0;
    bool persist_failed = false;  // the context could not be created: per-node path from then on
    bool persist_error = false;   // a launch gave up waiting (reported once)
    // GGML_MI355X_PERSIST_TIMING: HIP events around every eager persistent launch (not
    // under capture), summed at each status check
    bool persist_timing = false;
    hipEvent_t pt_ev[2] = {nullptr, nullptr};
    bool pt_pending = false;
    int64_t pt_launches = 0;
    double pt_ms = 0.0;
    bool graphs_on = true;  // GGML_MI355X_GRAPHS (replay of unchanged graphs)
    // captured replay of the last graph
    hipGraphExec_t gexec = nullptr;
    std::vector<uint64_t> signature;
    int same_calls = 0;
};

void set_device(int dev) { MI_HIP_CHECK(hipSetDevice(dev)); }

// ---- buffer iface

void buffer_free(ggml_backend_buffer_t buffer) {
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    set_device(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(ctx->dev_ptr);
    for (void *p : ctx->owned) (void)hipFree(p);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

void *buffer_get_base(ggml_backend_buffer_t buffer) { return ((BufferCtx *)buffer->context)->dev_ptr; }

enum ggml_status buffer_init_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor) {
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    if (tensor->view_src != nullptr) return GGML_STATUS_SUCCESS;
    const ggml_type fmt = side_fmt(tensor);
    if (fmt != GGML_TYPE_COUNT) {
        std::lock_guard<std::mutex> lk(ctx->mtx);
        auto ex = std::make_unique<TensorExtra>();
        ex->packed = (char *)tensor->data + side_offset(tensor);
        ex->fmt = fmt;
        tensor->extra = ex.get();
        ctx->extras.push_back(std::move(ex));
    }
    return GGML_STATUS_SUCCESS;
}

// Builds the side copy from the bytes at tensor->data: a re-layout of Q8_0 / Q4_0 blocks,
// or, for an F16 weight on the A8W8 path, W*diag(s) quantized to Q8_0 on the device
// (the reference quantizes on the host, patch:1674-1695).
void build_side_copy_locked(BufferCtx *ctx, ggml_tensor *tensor) {
    TensorExtra *ex = (TensorExtra *)tensor->extra;
    switch (tensor->type) {
        case GGML_TYPE_Q8_0:
            MI_K_CHECK(mi_prepack_q8_0(ctx->stream, tensor->data, ex->packed, tensor->ne[1], tensor->ne[0]));
            break;
        case GGML_TYPE_Q4_0:
            MI_K_CHECK(mi_prepack_q4_0(ctx->stream, tensor->data, ex->packed, tensor->ne[1], tensor->ne[0]));
            break;
        case GGML_TYPE_F16:
            MI_K_CHECK(mi_quantize_f16_q8_0(ctx->stream, (const uint16_t *)tensor->data, ex->s, ex->packed,
                                            tensor->ne[1], tensor->ne[0]));
            break;
        default:
            GGML_ABORT("MI355X: no side copy for %s weights", ggml_type_name(tensor->type));
    }
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    ex->ready = true;
}

void build_side_copy(BufferCtx *ctx, ggml_tensor *tensor) {
    std::lock_guard<std::mutex> lk(((TensorExtra *)tensor->extra)->mtx);
    build_side_copy_locked(ctx, tensor);
}

// a device copy of n fp32 factors, shared by every weight of the buffer with the same
// contents (the q/k/v projections share one SmoothQuant vector, gate/up another)
const float *upload_factors(BufferCtx *ctx, const float *v, int64_t n) {
    const std::string key((const char *)v, (size_t)n * sizeof(float));
    std::lock_guard<std::mutex> lk(ctx->mtx);
    auto it = ctx->factors_by_content.find(key);
    if (it != ctx->factors_by_content.end()) return (const float *)it->second;
    set_device(ctx->device);
    void *dev = nullptr;
    MI_HIP_CHECK(hipMalloc(&dev, (size_t)n * sizeof(float)));
    MI_HIP_CHECK(hipMemcpy(dev, v, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
    ctx->owned.push_back(dev);
    ctx->factors_by_content.emplace(key, dev);
    return (const float *)dev;
}

void buffer_set_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, const void *data, size_t offset,
                       size_t size) {
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipMemcpyAsync((char *)tensor->data + offset, data, size, hipMemcpyHostToDevice, ctx->stream));
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    if (!tensor->extra || tensor->view_src) return;

    const size_t total = ggml_nbytes(tensor);
    if (offset == 0 && size == total) {  // whole-tensor write
        build_side_copy(ctx, tensor);
        return;
    }
    // chunked write: count bytes per tensor, build the side copy once complete
    SetTracker *tr;
    {
        std::lock_guard<std::mutex> lk(ctx->mtx);
        auto &slot = ctx->trackers[tensor];
        if (!slot) {
            slot = std::make_unique<SetTracker>();
            slot->total_bytes = total;
        }
        tr = slot.get();
    }
    bool complete;
    {
        std::lock_guard<std::mutex> lk(tr->mtx);
        tr->bytes_written += size;
        complete = tr->bytes_written >= tr->total_bytes;
        if (complete) tr->bytes_written = 0;
    }
    if (complete) {
        build_side_copy(ctx, tensor);
        std::lock_guard<std::mutex> lk(ctx->mtx);
        ctx->trackers.erase(tensor);
    }
}

void buffer_get_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *tensor, void *data, size_t offset,
                       size_t size) {
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipMemcpyAsync(data, (const char *)tensor->data + offset, size, hipMemcpyDeviceToHost, ctx->stream));
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
}

void buffer_memset_tensor(ggml_backend_buffer_t buffer, ggml_tensor *tensor, uint8_t value, size_t offset,
                          size_t size) {
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipMemsetAsync((char *)tensor->data + offset, value, size, ctx->stream));
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
}

bool buffer_cpy_tensor(ggml_backend_buffer_t buffer, const ggml_tensor *src, ggml_tensor *dst) {
    if (!src->buffer || src->buffer->iface.get_base != buffer_get_base) return false;
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipMemcpyAsync(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice, ctx->stream));
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    if (dst->extra) build_side_copy(ctx, dst);
    return true;
}

void buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) {
    BufferCtx *ctx = (BufferCtx *)buffer->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipMemsetAsync(ctx->dev_ptr, value, ctx->size, ctx->stream));
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
}

const ggml_backend_buffer_i kBufferIface = {
    /* free_buffer   */ buffer_free,
    /* get_base      */ buffer_get_base,
    /* init_tensor   */ buffer_init_tensor,
    /* memset_tensor */ buffer_memset_tensor,
    /* set_tensor    */ buffer_set_tensor,
    /* get_tensor    */ buffer_get_tensor,
    /* cpy_tensor    */ buffer_cpy_tensor,
    /* clear         */ buffer_clear,
    /* reset         */ nullptr,
};

// ---- buffer type iface

const char *buft_get_name(ggml_backend_buffer_type_t buft) {
    return ((DeviceCtx *)buft->context)->buft_name.c_str();
}

ggml_backend_buffer_t buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    DeviceCtx *dctx = (DeviceCtx *)buft->context;
    set_device(dctx->device);
    BufferCtx *ctx = new BufferCtx();
    ctx->device = dctx->device;
    ctx->size = size;
    if (hipMalloc(&ctx->dev_ptr, size ? size : 256) != hipSuccess) {
        fprintf(stderr, "MI355X: hipMalloc of %zu bytes failed\n", size);
        delete ctx;
        return nullptr;
    }
    MI_HIP_CHECK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    return ggml_backend_buffer_init(buft, kBufferIface, ctx, size);
}

size_t buft_get_alignment(ggml_backend_buffer_type_t) { return 256; }
size_t buft_get_max_size(ggml_backend_buffer_type_t) { return SIZE_MAX; }

size_t buft_get_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor *tensor) {
    if (prepack_eligible(tensor)) return side_offset(tensor) + packed_size(tensor);
    return ggml_nbytes(tensor);
}

bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

const ggml_backend_buffer_type_i kBuftIface = {
    /* get_name       */ buft_get_name,
    /* alloc_buffer   */ buft_alloc_buffer,
    /* get_alignment  */ buft_get_alignment,
    /* get_max_size   */ buft_get_max_size,
    /* get_alloc_size */ buft_get_alloc_size,
    /* is_host        */ buft_is_host,
};

// ------------------------------------------------------------------ supports_op

bool is_f32_contig(const ggml_tensor *t) { return t && t->type == GGML_TYPE_F32 && ggml_is_contiguous(t); }
bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

bool supports_mul_mat(const ggml_tensor *op) {
    const ggml_tensor *a = op->src[0], *b = op->src[1];
    if (!is_f32_contig(b) || !is_f32_contig(op)) return false;
    if (b->ne[1] < 1 || b->ne[1] > 8 || b->ne[2] != 1 || b->ne[3] != 1) return false;
    if (a->ne[2] != 1 || a->ne[3] != 1) return false;
    // the planar side copy exists only for weights of this backend's buffers (a CPU
    // extra buffer type may hang its own data on tensor->extra)
    const bool owned = a->extra != nullptr && a->buffer && a->buffer->buft->iface.get_alloc_size == buft_get_alloc_size;
    switch (a->type) {
        case GGML_TYPE_Q8_0:
        case GGML_TYPE_Q4_0:
            return owned;
        case GGML_TYPE_F16:
            if (a->extra) return owned;  // quantized at upload (A8W8): the Q8_0 path
            return a->nb[0] == 2 && a->nb[1] % 16 == 0 && a->ne[0] % 8 == 0 && b->ne[0] * b->ne[1] * 2 <= 64 * 1024;
        default:
            return false;
    }
}

bool supports_fa(const ggml_tensor *op) {
    const ggml_tensor *q = op->src[0], *k = op->src[1], *v = op->src[2], *mask = op->src[3];
    const ggml_tensor *sinks = op->src[4], *kvl = op->src[5];
    float max_bias, softcap;
    memcpy(&max_bias, (const float *)op->op_params + 1, sizeof(float));
    memcpy(&softcap, (const float *)op->op_params + 2, sizeof(float));
    if (max_bias != 0.0f || softcap != 0.0f || sinks) return false;
    if (!q || q->type != GGML_TYPE_F32 || op->type != GGML_TYPE_F32 || !ggml_is_contiguous(op)) return false;
    // streams (ne[3]) are independent sequences with one query row each, or one stream
    // carries up to 8 query rows (ne[1]: a prompt ubatch, each row with its own mask row)
    const int64_t n_seq = q->ne[3], n_rows = q->ne[1];
    if (n_rows < 1 || n_rows > 8 || (n_rows > 1 && n_seq != 1)) return false;
    if (q->nb[0] != 4 || (q->ne[2] > 1 && q->nb[2] != (size_t)q->ne[0] * 4) || q->nb[3] % 4 || q->nb[1] % 4) return false;
    if (k->type != GGML_TYPE_F16 || v->type != GGML_TYPE_F16) return false;
    const int64_t d = q->ne[0];
    if ((d != 64 && d != 128) || k->ne[0] != d || v->ne[0] != d) return false;
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != n_seq || v->ne[3] != n_seq) return false;
    if (k->ne[2] < 1 || q->ne[2] % k->ne[2] != 0 || q->ne[2] / k->ne[2] > 8) return false;
    if (k->nb[0] != 2 || v->nb[0] != 2 || k->nb[1] % 16 || k->nb[2] % 16 || v->nb[1] % 16 || v->nb[2] % 16 ||
        (n_seq > 1 && (k->nb[3] % 16 || v->nb[3] % 16)))
        return false;
    // one mask row per sequence (or per query row), shared by the heads
    if (mask && (mask->type != GGML_TYPE_F16 || mask->ne[0] < k->ne[1] || mask->nb[0] != 2 || mask->ne[2] != 1 ||
                 mask->ne[1] < n_rows || (mask->ne[3] != 1 && mask->ne[3] != n_seq)))
        return false;
    if (kvl && (kvl->type != GGML_TYPE_I32 || !ggml_is_contiguous(kvl) || ggml_nelements(kvl) < n_seq)) return false;
    return true;
}

bool supports_op_impl(const ggml_tensor *op) {
    switch (op->op) {
        case GGML_OP_NONE:
        case GGML_OP_RESHAPE:
        case GGML_OP_VIEW:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:
            return true;
        case GGML_OP_MUL_MAT:
            return supports_mul_mat(op);
        case GGML_OP_FLASH_ATTN_EXT:
            return supports_fa(op);
        case GGML_OP_RMS_NORM:
            return is_f32_contig(op->src[0]) && is_f32_contig(op);
        case GGML_OP_ADD:
        case GGML_OP_MUL: {
            const ggml_tensor *a = op->src[0], *b = op->src[1];
            if (!is_f32_contig(a) || !is_f32_contig(b) || !is_f32_contig(op)) return false;
            return b->ne[0] == a->ne[0] && (ggml_nelements(b) == b->ne[0] || ggml_are_same_shape(a, b));
        }
        case GGML_OP_ROPE: {
            const int mode = op->op_params[2];
            float ext_factor;
            memcpy(&ext_factor, (const float *)op->op_params + 7, sizeof(float));
            return mode == GGML_ROPE_TYPE_NEOX && ext_factor == 0.0f && op->src[0]->type == GGML_TYPE_F32 &&
                   op->src[0]->nb[0] == 4 && op->src[2] == nullptr && op->src[1]->type == GGML_TYPE_I32 &&
                   is_f32_contig(op) && op->op_params[1] <= op->src[0]->ne[0];
        }
        case GGML_OP_SET_ROWS:
            return op->type == GGML_TYPE_F16 && op->nb[0] == 2 && op->src[0]->type == GGML_TYPE_F32 &&
                   op->src[0]->nb[0] == 4 && (op->src[1]->type == GGML_TYPE_I64 || op->src[1]->type == GGML_TYPE_I32) &&
                   op->src[0]->ne[2] == 1 && op->src[0]->ne[3] == 1;
        case GGML_OP_GET_ROWS:
            return (op->src[0]->type == GGML_TYPE_F16 || op->src[0]->type == GGML_TYPE_F32) &&
                   op->src[0]->nb[0] == ggml_type_size(op->src[0]->type) && op->src[1]->type == GGML_TYPE_I32 &&
                   ggml_is_contiguous(op->src[1]) && op->src[1]->ne[1] == 1 && is_f32_contig(op);
        case GGML_OP_GLU:
            return ggml_get_glu_op(op) == GGML_GLU_OP_SWIGLU && op->op_params[1] == 0 && is_f32_contig(op->src[0]) &&
                   is_f32_contig(op->src[1]) && is_f32_contig(op);
        case GGML_OP_ARGMAX:
            return is_f32_contig(op->src[0]) && op->type == GGML_TYPE_I32;
        default:
            return false;
    }
}

// ------------------------------------------------------------------ graph compute

bool is_noop(const ggml_tensor *t) {
    return t->op == GGML_OP_NONE || t->op == GGML_OP_RESHAPE || t->op == GGML_OP_VIEW || t->op == GGML_OP_PERMUTE ||
           t->op == GGML_OP_TRANSPOSE || ggml_is_empty(t);
}

const float *inv_s_of(const ggml_tensor *w) {
    const TensorExtra *ex = (const TensorExtra *)w->extra;
    return ex ? ex->inv_s : nullptr;
}

size_t fa_ws_need(const ggml_tensor *node) {
    const ggml_tensor *q = node->src[0], *k = node->src[1];
    return mi_fa_decode_batch_workspace_size(k->ne[1], q->ne[2], k->ne[2], q->ne[0], q->ne[3] * q->ne[1]);
}

size_t scratch_need(const ggml_tensor *node) {
    if (node->op == GGML_OP_MUL_MAT && packed_fmt(node->src[0]) == GGML_TYPE_Q8_0)
        return std::max(mi_mul_mat_q8_0_workspace_size(node->src[1]->ne[1], node->src[1]->ne[0]),
                        node->src[1]->ne[1] == 1 ? mi_xq_size(1, node->src[1]->ne[0]) : (size_t)0);
    if (node->op == GGML_OP_MUL_MAT && packed_fmt(node->src[0]) == GGML_TYPE_Q4_0)
        return mi_mul_mat_q4_0_workspace_size(node->src[1]->ne[1], node->src[1]->ne[0]);
    if (node->op == GGML_OP_ARGMAX)  // also the partials of the fused output head (try_fuse_norm_head)
        return std::max(mi_argmax_workspace_size(node->src[0]->ne[0], ggml_nrows(node->src[0])),
                        mi_head_f16_argmax_workspace_size(node->src[0]->ne[0], 4096));
    // one GLU row: fp16 (W4A16 down), or the A8W8 gate/up pair's quantized row and its
    // fp32 swiglu values
    if (node->op == GGML_OP_GLU && ggml_nrows(node) == 1)
        return mi_xq_size(1, ggml_nelements(node)) + GGML_PAD((size_t)ggml_nelements(node) * 4, 256);
    return 0;
}

void ensure_buffers(BackendCtx *ctx, ggml_cgraph *g) {
    size_t need_s = 0, need_fa = 0;
    int64_t need_c = 0;
    for (int i = 0; i < ggml_graph_n_nodes(g); i++) {
        ggml_tensor *n = ggml_graph_node(g, i);
        if (n->op == GGML_OP_FLASH_ATTN_EXT) need_fa = std::max(need_fa, fa_ws_need(n));
        if (n->op == GGML_OP_GLU && ggml_nrows(n) == 1) need_c = std::max(need_c, ggml_nelements(n) / 32);
        need_s = std::max(need_s, scratch_need(n));
    }
    if (need_c > ctx->ffn_counters_words) {
        if (ctx->ffn_counters) MI_HIP_CHECK(hipFree(ctx->ffn_counters));
        ctx->ffn_counters_words = GGML_PAD(need_c, 1024);
        MI_HIP_CHECK(hipMalloc(&ctx->ffn_counters, ctx->ffn_counters_words * 4));
        MI_HIP_CHECK(hipMemsetAsync(ctx->ffn_counters, 0, ctx->ffn_counters_words * 4, ctx->stream));
        MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
        ctx->signature.clear();
    }
    if (need_s > ctx->scratch_size) {
        if (ctx->scratch) MI_HIP_CHECK(hipFree(ctx->scratch));
        ctx->scratch_size = GGML_PAD(need_s, 1 << 20);
        MI_HIP_CHECK(hipMalloc(&ctx->scratch, ctx->scratch_size));
        ctx->signature.clear();
    }
    if (!ctx->rope_tab) MI_HIP_CHECK(hipMalloc(&ctx->rope_tab, 2 * 512 * sizeof(float)));
    if (need_fa > ctx->fa_ws_size) {
        if (ctx->fa_ws) MI_HIP_CHECK(hipFree(ctx->fa_ws));
        ctx->fa_ws_size = GGML_PAD(need_fa, 1 << 20);
        MI_HIP_CHECK(hipMalloc(&ctx->fa_ws, ctx->fa_ws_size));
        // the workspace's arrival counters must start at zero (kernels leave them zeroed)
        MI_HIP_CHECK(hipMemsetAsync(ctx->fa_ws, 0, ctx->fa_ws_size, ctx->stream));
        MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
        ctx->signature.clear();
    }
}

void run_mul_mat_q8_group(BackendCtx *ctx, ggml_tensor **nodes, int count) {
    const ggml_tensor *b = nodes[0]->src[1];
    const void *w[4];
    int64_t n[4];
    float *y[4];
    for (int i = 0; i < count; i++) {
        const TensorExtra *ex = (const TensorExtra *)nodes[i]->src[0]->extra;
        w[i] = ex->packed;
        n[i] = nodes[i]->src[0]->ne[1];
        y[i] = (float *)nodes[i]->data;
    }
    MI_K_CHECK(mi_mul_mat_q8_0_f32_multi(ctx->stream, count, w, n, y, b->ne[0], (const float *)b->data,
                                         inv_s_of(nodes[0]->src[0]), q8_rounding(), ctx->scratch,
                                         ctx->scratch_size));
}

void run_mul_mat(BackendCtx *ctx, ggml_tensor *node) {
    const ggml_tensor *a = node->src[0], *b = node->src[1];
    const int64_t n = a->ne[1], k = a->ne[0], m = b->ne[1];
    switch (packed_fmt(a)) {
        case GGML_TYPE_Q8_0: {
            const TensorExtra *ex = (const TensorExtra *)a->extra;
            GGML_ASSERT(ex && ex->ready && "Q8_0 / A8W8 weight used before its upload completed");
            MI_K_CHECK(mi_mul_mat_q8_0_f32(ctx->stream, ex->packed, (const float *)b->data, ex->inv_s,
                                           (float *)node->data, n, k, m, q8_rounding(), ctx->scratch,
                                           ctx->scratch_size));
            break;
        }
        case GGML_TYPE_Q4_0: {
            const TensorExtra *ex = (const TensorExtra *)a->extra;
            GGML_ASSERT(ex && ex->ready && "Q4_0 weight used before its upload completed");
            MI_K_CHECK(mi_mul_mat_q4_0_f32(ctx->stream, ex->packed, (const float *)b->data, (float *)node->data, n,
                                           k, m, ctx->scratch, ctx->scratch_size));
            break;
        }
        case GGML_TYPE_F16:
            MI_K_CHECK(mi_gemv_f16(ctx->stream, (const uint16_t *)a->data, (int64_t)(a->nb[1] / 2),
                                   (const float *)b->data, (float *)node->data, n, k, m));
            break;
        default:
            GGML_ABORT("MI355X: MUL_MAT with %s weights is not supported", ggml_type_name(a->type));
    }
}

void run_fa(BackendCtx *ctx, ggml_tensor *node) {
    const ggml_tensor *q = node->src[0], *k = node->src[1], *v = node->src[2], *mask = node->src[3];
    const ggml_tensor *kvl = node->src[5];
    float scale;
    memcpy(&scale, node->op_params, sizeof(float));
    if (q->ne[1] > 1) {  // one sequence's query rows: output [d, n_head, n_rows] contiguous
        MI_K_CHECK(mi_fa_decode_rows(ctx->stream, (const float *)q->data, k->data, v->data,
                                     mask ? (const uint16_t *)mask->data : nullptr,
                                     kvl ? (const int32_t *)kvl->data : nullptr, k->ne[1], q->ne[2], k->ne[2],
                                     q->ne[0], k->nb[1], k->nb[2], v->nb[1], v->nb[2], scale, (float *)node->data,
                                     q->ne[1], q->nb[1] / 4, mask ? mask->nb[1] / 2 : 0,
                                     (size_t)(q->ne[0] * q->ne[2]), ctx->fa_ws, ctx->fa_ws_size));
        return;
    }
    // output [d, n_head, 1, n_seq] contiguous; per-sequence strides of the inputs
    const size_t mask_seq = mask && mask->ne[3] > 1 ? mask->nb[3] / 2 : 0;
    MI_K_CHECK(mi_fa_decode_batch(ctx->stream, (const float *)q->data, k->data, v->data,
                                  mask ? (const uint16_t *)mask->data : nullptr,
                                  kvl ? (const int32_t *)kvl->data : nullptr, k->ne[1], q->ne[2], k->ne[2], q->ne[0],
                                  k->nb[1], k->nb[2], v->nb[1], v->nb[2], scale, (float *)node->data, q->ne[3],
                                  q->nb[3] / 4, k->nb[3], v->nb[3], mask_seq, (size_t)(q->ne[0] * q->ne[2]),
                                  ctx->fa_ws, ctx->fa_ws_size));
}

// ---- graph fusions
//
// Runs of adjacent nodes (no-op view nodes in between are skipped) that form one
// of the decode chains below run as one fused launch, as ggml-cuda fuses adjacent
// nodes.  A run is fused only when every intermediate tensor it does not write is
// read by nothing outside the run, so skipping those writes is unobservable.
//   attention input : RMS_NORM, MUL(w), MUL_MAT q/k/v, [ADD bias x3], ROPE q, ROPE k,
//                     SET_ROWS k, SET_ROWS v             -> mi_qkv_rope_kv_q8_0
//   normed matmuls  : RMS_NORM, MUL(w), MUL_MAT x1..4   -> mi_mul_mat_q8_0_f32_fused
//   matmul + add    : MUL_MAT, ADD(vector)              -> fused epilogue add
//   glu + matmul    : GLU swiglu, MUL_MAT, [ADD(vector)] -> mi_swiglu_quant_q8_0 +
//                                                          mi_gemv_q8_0_add
//   attention + o   : FLASH_ATTN_EXT, MUL_MAT, [ADD]     -> mi_fa_decode_partials +
//                                                          mi_mul_mat_q8_0_f32_lse
//   ubatch (Q4_0)   : [RMS_NORM, MUL(w)] MUL_MAT x1..4 [ADD bias each] or MUL_MAT
//                     ADD(residual), and GLU swiglu, MUL_MAT, [ADD] -> mi_mul_mat_q4_0_f32_batch
//   ubatch attn + o : FLASH_ATTN_EXT (n_seq rows), MUL_MAT (Q4_0), [ADD] -> mi_fa_decode_batch_q4act +
//                                                          mi_mul_mat_q4_0_batch_xp
//   ubatch FFN      : [RMS_NORM, MUL(w)] MUL_MAT gate, MUL_MAT up, GLU swiglu, MUL_MAT down,
//                     [ADD] -> mi_mul_mat_q4_0_gate_up_glu_batch + mi_mul_mat_q4_0_batch_xp
//   ubatch attn in  : [RMS_NORM, MUL(w)] MUL_MAT q/k/v, ADD bias x3, ROPE q, ROPE k, SET_ROWS k,
//                     SET_ROWS v -> mi_qkv_rope_kv_q4_0_batch
//   rope + kv write : ROPE q, ROPE k, SET_ROWS k, SET_ROWS v -> mi_rope_kv_rows

using Consumers = std::unordered_map<const ggml_tensor *, std::vector<const ggml_tensor *>>;

Consumers consumers_of(ggml_cgraph *g) {
    Consumers c;
    for (int i = 0; i < ggml_graph_n_nodes(g); i++) {
        const ggml_tensor *nd = ggml_graph_node(g, i);
        for (int s = 0; s < GGML_MAX_SRC; s++)
            if (nd->src[s]) c[nd->src[s]].push_back(nd);
    }
    return c;
}

bool is_view_op(const ggml_tensor *t) {
    return t->op == GGML_OP_RESHAPE || t->op == GGML_OP_VIEW || t->op == GGML_OP_PERMUTE || t->op == GGML_OP_TRANSPOSE;
}

// Stands for a reader outside the graph: a tensor flagged GGML_TENSOR_FLAG_OUTPUT (such as
// llama.cpp's result_norm, which it reads back as the embeddings) is consumed by the host
// after the graph ran, so a fusion must still write it.
const ggml_tensor kHostReader{};

// non-view consumers of t, looking through view nodes; kHostReader for an output tensor
void real_consumers(const Consumers &C, const ggml_tensor *t, std::vector<const ggml_tensor *> &out) {
    if (t->flags & GGML_TENSOR_FLAG_OUTPUT) out.push_back(&kHostReader);
    auto it = C.find(t);
    if (it == C.end()) return;
    for (const ggml_tensor *c : it->second) {
        if (is_view_op(c)) real_consumers(C, c, out);
        else out.push_back(c);
    }
}

bool only_consumed_by(const Consumers &C, const ggml_tensor *t, std::initializer_list<const ggml_tensor *> allowed) {
    std::vector<const ggml_tensor *> v;
    real_consumers(C, t, v);
    if (v.empty()) return false;
    for (const ggml_tensor *c : v) {
        bool ok = false;
        for (const ggml_tensor *a : allowed) ok = ok || c == a;
        if (!ok) return false;
    }
    return true;
}

// the tensor t aliases, through whole-tensor views (same bytes, no offset)
const ggml_tensor *alias_root(const ggml_tensor *t) {
    while (is_view_op(t) && t->src[0] && t->view_offs == 0 && ggml_nbytes(t) == ggml_nbytes(t->src[0]) &&
           ggml_is_contiguous(t) && ggml_is_contiguous(t->src[0]))
        t = t->src[0];
    return t;
}

int next_real(ggml_cgraph *g, int i) {
    const int nn = ggml_graph_n_nodes(g);
    while (i < nn && is_noop(ggml_graph_node(g, i))) i++;
    return i;
}

// byte ranges of a and b intersect (ggml's allocator may place a node's output in the
// memory of an input whose last consumer ran before it: a fused launch that still reads
// that input from other workgroups while writing the output must not run then)
bool overlaps(const ggml_tensor *a, const ggml_tensor *b) {
    const uintptr_t a0 = (uintptr_t)a->data, a1 = a0 + ggml_nbytes(a);
    const uintptr_t b0 = (uintptr_t)b->data, b1 = b0 + ggml_nbytes(b);
    return a0 < b1 && b0 < a1;
}

bool is_row_vector(const ggml_tensor *t, int64_t n) {
    return t && is_f32_contig(t) && ggml_nelements(t) == n && aligned16(t->data);
}

// a Q8_0 or Q4_0 MUL_MAT (type t) on one activation row with the prepacked side copy ready
bool gemv_node(const ggml_tensor *n, ggml_type t) {
    if (n->op != GGML_OP_MUL_MAT) return false;
    const ggml_tensor *a = n->src[0], *b = n->src[1];
    const TensorExtra *ex = (const TensorExtra *)a->extra;
    return ex && ex->fmt == t && ex->ready && b->type == GGML_TYPE_F32 && ggml_nrows(b) == 1 &&
           ggml_is_contiguous(b) && aligned16(b->data) && is_f32_contig(n);
}
bool q8_gemv_node(const ggml_tensor *n) { return gemv_node(n, GGML_TYPE_Q8_0); }

// the weight format of a fusable one-row MUL_MAT, or GGML_TYPE_COUNT
ggml_type gemv_type(const ggml_tensor *n) {
    if (gemv_node(n, GGML_TYPE_Q8_0)) return GGML_TYPE_Q8_0;
    if (gemv_node(n, GGML_TYPE_Q4_0)) return GGML_TYPE_Q4_0;
    return GGML_TYPE_COUNT;
}

bool rms_mul_head(ggml_cgraph *g, int i, const Consumers &C, int &j, const ggml_tensor *&x, const ggml_tensor *&nw,
                  const ggml_tensor *&mul, float &eps) {
    const ggml_tensor *rms = ggml_graph_node(g, i);
    if (rms->op != GGML_OP_RMS_NORM) return false;
    x = rms->src[0];
    if (!is_f32_contig(x) || ggml_nrows(x) != 1 || x->ne[0] % 32 || x->ne[0] > 4096 || !aligned16(x->data)) return false;
    memcpy(&eps, rms->op_params, sizeof(float));
    j = next_real(g, i + 1);
    if (j >= ggml_graph_n_nodes(g)) return false;
    mul = ggml_graph_node(g, j);
    if (mul->op != GGML_OP_MUL || mul->src[0] != rms || !is_row_vector(mul->src[1], x->ne[0])) return false;
    if (!only_consumed_by(C, rms, {mul})) return false;
    nw = mul->src[1];
    return true;
}

// the rotation table for (pos tensor, head_dim, rope parameters), built on the stream at
// its first use in this graph run
const float *rope_table_for(BackendCtx *ctx, const void *pos, int64_t hd, float freq_base, float freq_scale,
                            float attn_factor) {
    if (!ctx->rope_tab || hd > 1024) return nullptr;
    auto &k = ctx->rope_key;
    if (k.valid && k.pos == pos && k.hd == hd && k.freq_base == freq_base && k.freq_scale == freq_scale &&
        k.attn_factor == attn_factor)
        return ctx->rope_tab;
    MI_K_CHECK(mi_rope_table(ctx->stream, (const int32_t *)pos, hd, freq_base, freq_scale, attn_factor,
                             ctx->rope_tab));
    k.pos = pos;
    k.hd = hd;
    k.freq_base = freq_base;
    k.freq_scale = freq_scale;
    k.attn_factor = attn_factor;
    k.valid = true;
    return ctx->rope_tab;
}

// The attention-input chain of one token: RMS_NORM, MUL(w), MUL_MAT q/k/v (one activation
// row, Q8_0 or Q4_0), [ADD bias x3], ROPE q, ROPE k, SET_ROWS k, SET_ROWS v.
struct AttnInMatch {
    int end = -1;  // index of the last node (SET_ROWS v)
    const ggml_tensor *x = nullptr, *nw = nullptr, *mul = nullptr;
    float eps = 0.0f;
    const ggml_tensor *mm[3] = {}, *out[3] = {}, *bias[3] = {}, *rope[2] = {}, *sr[2] = {};
    ggml_type wt = GGML_TYPE_COUNT;
    int64_t hd = 0;
};

bool match_attn_in(ggml_cgraph *g, int i, const Consumers &C, AttnInMatch &M) {
    const int nn = ggml_graph_n_nodes(g);
    int j;
    if (!rms_mul_head(g, i, C, j, M.x, M.nw, M.mul, M.eps)) return false;
    const ggml_tensor *const *mm = M.mm;
    for (int t = 0; t < 3; t++) {
        j = next_real(g, j + 1);
        if (j >= nn) return false;
        M.mm[t] = ggml_graph_node(g, j);
        if (t == 0) M.wt = gemv_type(M.mm[0]);
        if (M.wt == GGML_TYPE_COUNT || !gemv_node(mm[t], M.wt) || mm[t]->src[1] != M.mul ||
            inv_s_of(mm[t]->src[0]) != inv_s_of(mm[0]->src[0]))
            return false;
        M.out[t] = mm[t];
    }
    if (!only_consumed_by(C, M.mul, {mm[0], mm[1], mm[2]})) return false;
    int jb = next_real(g, j + 1);
    if (jb < nn && ggml_graph_node(g, jb)->op == GGML_OP_ADD) {
        for (int t = 0; t < 3; t++) {
            if (jb >= nn) return false;
            const ggml_tensor *ad = ggml_graph_node(g, jb);
            if (ad->op != GGML_OP_ADD || ad->src[0] != mm[t] || !is_row_vector(ad->src[1], mm[t]->ne[0]) ||
                !is_f32_contig(ad) || !only_consumed_by(C, mm[t], {ad}))
                return false;
            M.bias[t] = ad->src[1];
            M.out[t] = ad;
            j = jb;
            jb = next_real(g, jb + 1);
        }
    }
    const ggml_tensor *const *rope = M.rope;
    for (int t = 0; t < 2; t++) {
        j = next_real(g, j + 1);
        if (j >= nn) return false;
        M.rope[t] = ggml_graph_node(g, j);
        if (rope[t]->op != GGML_OP_ROPE || !supports_op_impl(rope[t]) || alias_root(rope[t]->src[0]) != M.out[t] ||
            !only_consumed_by(C, M.out[t], {rope[t]}))
            return false;
    }
    const ggml_tensor *r = rope[0];
    const int64_t hd = r->src[0]->ne[0];
    M.hd = hd;
    if (r->op_params[1] != hd || rope[1]->op_params[1] != hd || rope[1]->src[0]->ne[0] != hd || hd % 16 ||
        rope[1]->src[1] != r->src[1] || ggml_nelements(r->src[1]) != 1 ||
        memcmp(r->op_params + 5, rope[1]->op_params + 5, 4 * sizeof(int32_t)) != 0 ||
        mm[0]->ne[0] % hd || mm[1]->ne[0] % hd || !is_f32_contig(rope[0]))
        return false;
    if (M.wt == GGML_TYPE_Q4_0 && (hd > 128 || mm[2]->ne[0] % 2)) return false;
    const ggml_tensor *const *sr = M.sr;
    for (int t = 0; t < 2; t++) {
        j = next_real(g, j + 1);
        if (j >= nn) return false;
        M.sr[t] = ggml_graph_node(g, j);
        const ggml_tensor *src = t == 0 ? rope[1] : M.out[2];
        if (sr[t]->op != GGML_OP_SET_ROWS || !supports_op_impl(sr[t]) || alias_root(sr[t]->src[0]) != src ||
            ggml_nrows(sr[t]->src[0]) != 1 || sr[t]->src[0]->ne[0] != mm[t + 1]->ne[0] ||
            ggml_nelements(sr[t]->src[1]) != 1 || (t == 1 && sr[1]->src[1] != sr[0]->src[1]))
            return false;
    }
    if (!only_consumed_by(C, rope[1], {sr[0]}) || !only_consumed_by(C, M.out[2], {sr[1]})) return false;
    if (overlaps(rope[0], M.x) || overlaps(rope[0], M.nw)) return false;
    M.end = j;
    return true;
}

void rope_params(const ggml_tensor *r, float &freq_base, float &freq_scale, float &attn_factor) {
    memcpy(&freq_base, (const float *)r->op_params + 5, sizeof(float));
    memcpy(&freq_scale, (const float *)r->op_params + 6, sizeof(float));
    memcpy(&attn_factor, (const float *)r->op_params + 8, sizeof(float));
}

int try_fuse_attn_in(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    AttnInMatch M;
    if (!match_attn_in(g, i, C, M)) return 0;
    const ggml_tensor *const *mm = M.mm, *const *sr = M.sr;
    const ggml_tensor *r = M.rope[0];
    const int64_t hd = M.hd;
    const void *w[3];
    int64_t n[3];
    const float *bp[3];
    for (int t = 0; t < 3; t++) {
        w[t] = ((const TensorExtra *)mm[t]->src[0]->extra)->packed;
        n[t] = mm[t]->src[0]->ne[1];
        bp[t] = M.bias[t] ? (const float *)M.bias[t]->data : nullptr;
    }
    float freq_base, freq_scale, attn_factor;
    rope_params(r, freq_base, freq_scale, attn_factor);
    const ggml_tensor *idx = sr[0]->src[1];
    const float *tab = rope_table_for(ctx, r->src[1]->data, hd, freq_base, freq_scale, attn_factor);
    if (M.wt == GGML_TYPE_Q4_0) {
        MI_K_CHECK(mi_qkv_rope_kv_q4_0(ctx->stream, w, n, bp, M.x->ne[0], (const float *)M.x->data,
                                       (const float *)M.nw->data, M.eps, hd, (const int32_t *)r->src[1]->data,
                                       freq_base, freq_scale, attn_factor, (float *)M.rope[0]->data, sr[0]->data,
                                       sr[0]->nb[1], sr[1]->data, sr[1]->nb[1], idx->data,
                                       idx->type == GGML_TYPE_I64, std::min(sr[0]->ne[1], sr[1]->ne[1]), tab));
        return M.end + 1 - i;
    }
    MI_K_CHECK(mi_qkv_rope_kv_q8_0(ctx->stream, w, n, bp, M.x->ne[0], (const float *)M.x->data,
                                   (const float *)M.nw->data, M.eps, inv_s_of(mm[0]->src[0]), q8_rounding(), hd,
                                   (const int32_t *)r->src[1]->data, freq_base, freq_scale, attn_factor,
                                   (float *)M.rope[0]->data, sr[0]->data, sr[0]->nb[1], sr[1]->data, sr[1]->nb[1],
                                   idx->data, idx->type == GGML_TYPE_I64, std::min(sr[0]->ne[1], sr[1]->ne[1]),
                                   tab));
    return M.end + 1 - i;
}

const ggml_tensor *matmul_add_tail(ggml_cgraph *g, int j, const ggml_tensor *mm, const Consumers &C,
                                   const ggml_tensor *&vec);

// W4A16 FFN: [norm] -> gate, up (mm[0], mm[1], nodes up to index last) -> GLU swiglu ->
// down MUL_MAT [-> ADD residual]: the GLU output goes to scratch as fp16 (the conversion
// the down projection's MUL_MAT applies to its src1), so the chain is two launches.
int try_fuse_gate_up_down_q4(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C, int last,
                             const ggml_tensor *const *mm, const ggml_tensor *x, const ggml_tensor *nw, float eps) {
    const int nn = ggml_graph_n_nodes(g);
    const int jg = next_real(g, last + 1);
    if (jg >= nn) return 0;
    const ggml_tensor *glu = ggml_graph_node(g, jg);
    if (glu->op != GGML_OP_GLU || !supports_op_impl(glu) || glu->src[0] != mm[0] || glu->src[1] != mm[1] ||
        mm[0]->ne[0] != mm[1]->ne[0] || !only_consumed_by(C, mm[0], {glu}) || !only_consumed_by(C, mm[1], {glu}))
        return 0;
    const int jd = next_real(g, jg + 1);
    if (jd >= nn) return 0;
    const ggml_tensor *down = ggml_graph_node(g, jd);
    const int64_t nf = mm[0]->ne[0];
    if (!gemv_node(down, GGML_TYPE_Q4_0) || down->src[1] != glu || !only_consumed_by(C, glu, {down}) ||
        down->src[0]->ne[0] != nf || nf / 32 > 1024 || ctx->scratch_size < (size_t)nf * 2)
        return 0;
    const ggml_tensor *vec = nullptr;
    const ggml_tensor *ad = matmul_add_tail(g, jd, down, C, vec);
    uint16_t *h = (uint16_t *)ctx->scratch;
    MI_K_CHECK(mi_gate_up_swiglu_q4_0(ctx->stream, ((const TensorExtra *)mm[0]->src[0]->extra)->packed,
                                      ((const TensorExtra *)mm[1]->src[0]->extra)->packed, nf, x->ne[0],
                                      (const float *)x->data, nw ? (const float *)nw->data : nullptr, eps, h));
    MI_K_CHECK(mi_gemv_q4_0_f16_add(ctx->stream, ((const TensorExtra *)down->src[0]->extra)->packed, h,
                                    ad ? (const float *)vec->data : nullptr, (float *)(ad ? ad->data : down->data),
                                    down->src[0]->ne[1], nf, 1));
    return (ad ? next_real(g, jd + 1) : jd) + 1 - i;
}

// A8W8 FFN: [norm] -> gate, up -> GLU swiglu -> down MUL_MAT [-> ADD residual] in two
// launches (MI_FFN_PAIR; 0 keeps the three of fused gate/up, swiglu-quantize, down):
//   default: the gate/up launch pairs 8 gate rows with the same 8 up rows per workgroup
//     (its 1120-workgroup grid at the 1.5B shape), and the last of the four workgroups of
//     each 32-block quantizes it (per-block arrival counters), so the down launch is
//     unchanged and the swiglu-quantize launch is gone;
//   f32: the pair writes the swiglu values in fp32 and the down launch quantizes them in
//     its prologue (mi_mul_mat_q8_0_f32_fused without norm): measured 1,028 against 1,044
//     tok/s for the three launches (every down workgroup reads and quantizes 35 KB).
// MI_FUSE_GU_SWIGLU=1 instead quantizes in the gate/up epilogue with whole 32-row blocks
// per workgroup: 280 workgroups on 256 CUs at the 1.5B shape, 10.9 us against 8.2 + 2.6 us.
int try_fuse_gate_up_down_q8(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C, int last,
                             const ggml_tensor *const *mm, const ggml_tensor *x, const ggml_tensor *nw, float eps) {
    static const bool blocks = env_flag("MI_FUSE_GU_SWIGLU", false);
    static const int pair = [] {  // 0 off, 1 fp32 + down prologue, 2 last-arrival quantization
        const char *e = getenv("MI_FFN_PAIR");
        if (!e || !*e) return 2;
        if (e[0] == '0') return 0;
        return strcmp(e, "f32") == 0 ? 1 : 2;
    }();
    if (!blocks && !pair) return 0;
    const int nn = ggml_graph_n_nodes(g);
    const int jg = next_real(g, last + 1);
    if (jg >= nn) return 0;
    const ggml_tensor *glu = ggml_graph_node(g, jg);
    if (glu->op != GGML_OP_GLU || !supports_op_impl(glu) || glu->src[0] != mm[0] || glu->src[1] != mm[1] ||
        mm[0]->ne[0] != mm[1]->ne[0] || !only_consumed_by(C, mm[0], {glu}) || !only_consumed_by(C, mm[1], {glu}))
        return 0;
    const int jd = next_real(g, jg + 1);
    if (jd >= nn) return 0;
    const ggml_tensor *down = ggml_graph_node(g, jd);
    const int64_t nf = mm[0]->ne[0], k = x->ne[0];
    if (!q8_gemv_node(down) || down->src[1] != glu || !only_consumed_by(C, glu, {down}) || down->src[0]->ne[0] != nf ||
        k > 2048)
        return 0;
    const ggml_tensor *vec = nullptr;
    const ggml_tensor *ad = matmul_add_tail(g, jd, down, C, vec);
    const TensorExtra *exd = (const TensorExtra *)down->src[0]->extra;
    const void *wg = ((const TensorExtra *)mm[0]->src[0]->extra)->packed;
    const void *wu = ((const TensorExtra *)mm[1]->src[0]->extra)->packed;
    const float *xf = (const float *)x->data, *nwf = nw ? (const float *)nw->data : nullptr;
    float *yd = (float *)(ad ? ad->data : down->data);
    const float *addv = ad ? (const float *)vec->data : nullptr;
    if (blocks) {
        if (nf % 32 || ctx->scratch_size < mi_xq_size(1, nf)) return 0;
        MI_K_CHECK(mi_gate_up_swiglu_q8_0(ctx->stream, wg, wu, nf, k, xf, nwf, eps, inv_s_of(mm[0]->src[0]),
                                          exd->inv_s, q8_rounding(), ctx->scratch));
        MI_K_CHECK(mi_gemv_q8_0_add(ctx->stream, exd->packed, ctx->scratch, addv, yd, down->src[0]->ne[1], nf, 1));
    } else if (pair == 2) {
        const size_t hoff = mi_xq_size(1, nf);
        if (nf % 32 || ctx->scratch_size < hoff + (size_t)nf * 4 || ctx->ffn_counters_words < nf / 32) return 0;
        MI_K_CHECK(mi_gate_up_pair_q8_0(ctx->stream, wg, wu, nf, k, xf, nwf, eps, inv_s_of(mm[0]->src[0]), exd->inv_s,
                                        q8_rounding(), ctx->scratch, (float *)((uint8_t *)ctx->scratch + hoff),
                                        ctx->ffn_counters));
        MI_K_CHECK(mi_gemv_q8_0_add(ctx->stream, exd->packed, ctx->scratch, addv, yd, down->src[0]->ne[1], nf, 1));
    } else {
        // the down launch quantizes h in its prologue: n_ff <= 12288
        if (nf % 32 || nf > 12288 || ctx->scratch_size < (size_t)nf * 4) return 0;
        float *h = (float *)ctx->scratch;
        MI_K_CHECK(mi_gate_up_swiglu_f32_q8_0(ctx->stream, wg, wu, nf, k, xf, nwf, eps, inv_s_of(mm[0]->src[0]),
                                              exd->inv_s, q8_rounding(), h));
        const void *wdn = exd->packed;
        const int64_t nd = down->src[0]->ne[1];
        MI_K_CHECK(mi_mul_mat_q8_0_f32_fused(ctx->stream, 1, &wdn, &nd, &yd, &addv, nf, h, nullptr, 0.0f, nullptr,
                                             q8_rounding()));
    }
    return (ad ? next_real(g, jd + 1) : jd) + 1 - i;
}

int try_fuse_norm_matmuls(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    const int nn = ggml_graph_n_nodes(g);
    int j;
    const ggml_tensor *x, *nw, *mul;
    float eps;
    if (!rms_mul_head(g, i, C, j, x, nw, mul, eps)) return 0;
    const ggml_tensor *mm[4] = {nullptr, nullptr, nullptr, nullptr};
    int cnt = 0, last = j;
    ggml_type wt = GGML_TYPE_COUNT;
    for (int jj = next_real(g, j + 1); jj < nn && cnt < 4; jj = next_real(g, jj + 1)) {
        const ggml_tensor *nd = ggml_graph_node(g, jj);
        if (cnt == 0) wt = gemv_type(nd);
        if (wt == GGML_TYPE_COUNT || !gemv_node(nd, wt) || nd->src[1] != mul ||
            inv_s_of(nd->src[0]) != inv_s_of(mm[0] ? mm[0]->src[0] : nd->src[0]))
            break;
        mm[cnt++] = nd;
        last = jj;
    }
    if (cnt == 0) return 0;
    for (int t = 0; t < cnt; t++)
        if (overlaps(mm[t], x) || overlaps(mm[t], nw)) return 0;
    std::vector<const ggml_tensor *> cons;
    real_consumers(C, mul, cons);
    for (const ggml_tensor *c : cons) {
        bool in = false;
        for (int t = 0; t < cnt; t++) in = in || c == mm[t];
        if (!in) return 0;
    }
    const void *w[4];
    int64_t n[4];
    float *y[4];
    for (int t = 0; t < cnt; t++) {
        w[t] = ((const TensorExtra *)mm[t]->src[0]->extra)->packed;
        n[t] = mm[t]->src[0]->ne[1];
        y[t] = (float *)mm[t]->data;
    }
    if (wt == GGML_TYPE_Q4_0) {
        if (cnt == 2) {
            if (int used = try_fuse_gate_up_down_q4(ctx, g, i, C, last, mm, x, nw, eps)) return used;
        }
        MI_K_CHECK(mi_mul_mat_q4_0_f32_fused(ctx->stream, cnt, w, n, y, nullptr, x->ne[0], (const float *)x->data,
                                             (const float *)nw->data, eps));
        return last + 1 - i;
    }
    if (cnt == 2) {
        if (int used = try_fuse_gate_up_down_q8(ctx, g, i, C, last, mm, x, nw, eps)) return used;
    }
    MI_K_CHECK(mi_mul_mat_q8_0_f32_fused(ctx->stream, cnt, w, n, y, nullptr, x->ne[0], (const float *)x->data,
                                         (const float *)nw->data, eps, inv_s_of(mm[0]->src[0]), q8_rounding()));
    return last + 1 - i;
}

// MUL_MAT (Q8_0, one row) followed by its only consumer ADD(mm, v) with a vector of the
// output length; returns the ADD node and the vector
const ggml_tensor *matmul_add_tail(ggml_cgraph *g, int j, const ggml_tensor *mm, const Consumers &C,
                                   const ggml_tensor *&vec) {
    const int k = next_real(g, j + 1);
    if (k >= ggml_graph_n_nodes(g)) return nullptr;
    const ggml_tensor *ad = ggml_graph_node(g, k);
    if (ad->op != GGML_OP_ADD || !is_f32_contig(ad) || ggml_nelements(ad) != mm->ne[0]) return nullptr;
    const ggml_tensor *other = ad->src[0] == mm ? ad->src[1] : (ad->src[1] == mm ? ad->src[0] : nullptr);
    if (!other || other == mm || !is_row_vector(other, mm->ne[0]) || !only_consumed_by(C, mm, {ad})) return nullptr;
    vec = other;
    return ad;
}

// RMS_NORM -> MUL(norm_w) -> MUL_MAT(F16 weight, one row) -> ARGMAX: the output head of
// a decode token in one launch with the norm in its prologue and the argmax's first pass
// in its epilogue, then the argmax's final pass (the logits are written as the MUL_MAT
// node's output)
int try_fuse_norm_head(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    int j;
    const ggml_tensor *x, *nw, *mul;
    float eps;
    if (!rms_mul_head(g, i, C, j, x, nw, mul, eps)) return 0;
    const int nn = ggml_graph_n_nodes(g);
    const int jm = next_real(g, j + 1);
    if (jm >= nn) return 0;
    ggml_tensor *mm = ggml_graph_node(g, jm);
    if (mm->op != GGML_OP_MUL_MAT || mm->src[1] != mul || !is_f32_contig(mm) || !only_consumed_by(C, mul, {mm}))
        return 0;
    const ggml_tensor *a = mm->src[0];
    if (a->type != GGML_TYPE_F16 || a->nb[0] != 2 || a->nb[1] % 16 || !aligned16(a->data) || a->ne[0] != x->ne[0] ||
        a->ne[2] != 1 || a->ne[3] != 1 || !aligned16(nw->data))
        return 0;
    const int ja = next_real(g, jm + 1);
    if (ja >= nn) return 0;
    ggml_tensor *am = ggml_graph_node(g, ja);
    if (am->op != GGML_OP_ARGMAX || am->src[0] != mm) return 0;
    const int64_t n = a->ne[1], k = a->ne[0];
    if (ctx->scratch_size < mi_head_f16_argmax_workspace_size(n, k)) return 0;
    MI_K_CHECK(mi_head_f16_argmax(ctx->stream, (const uint16_t *)a->data, (int64_t)(a->nb[1] / 2),
                                  (const float *)x->data, (const float *)nw->data, eps, (float *)mm->data,
                                  (int32_t *)am->data, n, k, ctx->scratch, ctx->scratch_size));
    return ja + 1 - i;
}

int try_fuse_matmul_add(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    const ggml_tensor *mm = ggml_graph_node(g, i);
    const ggml_type wt = gemv_type(mm);
    if (wt == GGML_TYPE_COUNT) return 0;
    const int64_t k = mm->src[0]->ne[0];
    if (wt == GGML_TYPE_Q4_0 && k / 32 > 1008) return 0;
    const ggml_tensor *vec = nullptr;
    const ggml_tensor *ad = matmul_add_tail(g, i, mm, C, vec);
    if (!ad) return 0;
    // one launch reads the whole activation in every workgroup and writes the sum
    if ((wt == GGML_TYPE_Q4_0 || k <= 4096) && overlaps(ad, mm->src[1])) return 0;
    const TensorExtra *ex = (const TensorExtra *)mm->src[0]->extra;
    const void *w = ex->packed;
    const int64_t n = mm->src[0]->ne[1];
    float *y = (float *)ad->data;
    const float *add = (const float *)vec->data;
    if (wt == GGML_TYPE_Q4_0) {
        MI_K_CHECK(mi_mul_mat_q4_0_f32_fused(ctx->stream, 1, &w, &n, &y, &add, k, (const float *)mm->src[1]->data,
                                             nullptr, 0.0f));
    } else if (k <= 4096) {
        MI_K_CHECK(mi_mul_mat_q8_0_f32_fused(ctx->stream, 1, &w, &n, &y, &add, k, (const float *)mm->src[1]->data,
                                             nullptr, 0.0f, ex->inv_s, q8_rounding()));
    } else {
        GGML_ASSERT(ctx->scratch_size >= mi_xq_size(1, k));
        MI_K_CHECK(mi_act_quant_q8_0(ctx->stream, (const float *)mm->src[1]->data, ex->inv_s, 1, k, ctx->scratch,
                                     q8_rounding()));
        MI_K_CHECK(mi_gemv_q8_0_add(ctx->stream, w, ctx->scratch, add, y, n, k, 1));
    }
    return next_real(g, i + 1) + 1 - i;
}

int try_fuse_glu_matmul(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    const ggml_tensor *glu = ggml_graph_node(g, i);
    if (glu->op != GGML_OP_GLU || !supports_op_impl(glu) || !glu->src[1] || ggml_nrows(glu) != 1 ||
        !aligned16(glu->src[0]->data) || !aligned16(glu->src[1]->data))
        return 0;
    const int j = next_real(g, i + 1);
    if (j >= ggml_graph_n_nodes(g)) return 0;
    const ggml_tensor *mm = ggml_graph_node(g, j);
    if (!q8_gemv_node(mm) || mm->src[1] != glu || !only_consumed_by(C, glu, {mm})) return 0;
    const int64_t k = mm->src[0]->ne[0];
    if (ctx->scratch_size < mi_xq_size(1, k)) return 0;
    const TensorExtra *ex = (const TensorExtra *)mm->src[0]->extra;
    const ggml_tensor *vec = nullptr;
    const ggml_tensor *ad = matmul_add_tail(g, j, mm, C, vec);
    MI_K_CHECK(mi_swiglu_quant_q8_0(ctx->stream, (const float *)glu->src[0]->data, (const float *)glu->src[1]->data,
                                    ex->inv_s, k, ctx->scratch, q8_rounding()));
    MI_K_CHECK(mi_gemv_q8_0_add(ctx->stream, ex->packed, ctx->scratch, ad ? (const float *)vec->data : nullptr,
                                (float *)(ad ? ad->data : mm->data), mm->src[0]->ne[1], k, 1));
    return (ad ? next_real(g, j + 1) : j) + 1 - i;
}

// FLASH_ATTN_EXT (one token, one sequence) whose output only feeds a Q8_0 projection
// [+ ADD]: the attention leaves its splits' records in the FA workspace and the
// projection merges them in its prologue (no combine launch, no attention-output write).
// Opt-in (MI_FUSE_FA_O=1): every projection workgroup then reads all splits' records
// (12 splits x 12 heads x 528 B at a 768-row KV view), which measured slower than the
// separate combine launch on the Qwen2.5-1.5B shape (6.97 us against 3.45 + 3.17 us).
int try_fuse_fa_o(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    static const bool on = env_flag("MI_FUSE_FA_O", false);
    if (!on) return 0;
    const ggml_tensor *fa = ggml_graph_node(g, i);
    const ggml_tensor *q = fa->src[0], *k = fa->src[1], *v = fa->src[2], *mask = fa->src[3];
    if (q->ne[1] != 1 || q->ne[3] != 1 || !ggml_is_contiguous(fa)) return 0;
    const int64_t d = q->ne[0], n_head = q->ne[2];
    const int j = next_real(g, i + 1);
    if (j >= ggml_graph_n_nodes(g)) return 0;
    const ggml_tensor *mm = ggml_graph_node(g, j);
    if (!q8_gemv_node(mm) || alias_root(mm->src[1]) != fa || !only_consumed_by(C, fa, {mm})) return 0;
    const int64_t kk = mm->src[0]->ne[0];
    if (kk != d * n_head || kk > 2048 || d % 4) return 0;
    const int64_t S = mi_fa_decode_num_splits(k->ne[1], n_head, k->ne[2], d);
    if (S < 1 || S > 16) return 0;
    if (ctx->fa_ws_size < mi_fa_decode_workspace_size(k->ne[1], n_head, k->ne[2], d)) return 0;
    const ggml_tensor *vec = nullptr;
    const ggml_tensor *ad = matmul_add_tail(g, j, mm, C, vec);
    float scale;
    memcpy(&scale, fa->op_params, sizeof(float));
    const ggml_tensor *kvl = fa->src[5];
    MI_K_CHECK(mi_fa_decode_partials(ctx->stream, (const float *)q->data, k->data, v->data,
                                     mask ? (const uint16_t *)mask->data : nullptr,
                                     kvl ? (const int32_t *)kvl->data : nullptr, k->ne[1], n_head, k->ne[2], d,
                                     k->nb[1], k->nb[2], v->nb[1], v->nb[2], scale, ctx->fa_ws, ctx->fa_ws_size));
    const TensorExtra *ex = (const TensorExtra *)mm->src[0]->extra;
    MI_K_CHECK(mi_mul_mat_q8_0_f32_lse(ctx->stream, ex->packed, mm->src[0]->ne[1], (float *)(ad ? ad->data : mm->data),
                                       ad ? (const float *)vec->data : nullptr, (const float *)ctx->fa_ws, S, n_head,
                                       d, ex->inv_s, q8_rounding()));
    return (ad ? next_real(g, j + 1) : j) + 1 - i;
}

// ---- the whole layer stack of one A8W8 token as one persistent launch
//
// A decoder layer of the one-token graph:
//   attention input (match_attn_in, Q8_0), FLASH_ATTN_EXT (q = the rotated q, K / V = the
//   views of the caches the SET_ROWS wrote, an optional F16 mask row), MUL_MAT o (Q8_0), ADD(o, x),
//   RMS_NORM, MUL(w), MUL_MAT gate, MUL_MAT up, GLU swiglu, MUL_MAT down, ADD(down, x1)
// with every intermediate read by nothing outside the layer.  A run of such layers, each
// reading the previous one's output, with one position / cache row / attention view /
// mask, runs as mi_persist_decode_q8_0 (GGML_MI355X_PERSIST=1).
struct PersistLayerMatch {
    int end = -1;  // the layer's last node (the FFN residual ADD)
    const ggml_tensor *x = nullptr, *out = nullptr, *rms = nullptr, *x1 = nullptr;
    const ggml_tensor *rope = nullptr, *idx = nullptr, *kvl = nullptr, *fa = nullptr;
    const void *mask = nullptr;  // the F16 mask row's data, or null
    mi_persist_layer L{};
    float eps = 0.0f, eps_ffn = 0.0f, kq_scale = 0.0f;
    int64_t n_embd = 0, n_head = 0, n_head_kv = 0, hd = 0, n_ff = 0, n_kv = 0, n_cache_rows = 0;
    size_t kv_row_bytes = 0;
};


// ADD(a, b) in either operand order, one row of n floats
bool is_add_of(const ggml_tensor *ad, const ggml_tensor *a, const ggml_tensor *b, int64_t n) {
    return ad->op == GGML_OP_ADD && is_f32_contig(ad) && ggml_nelements(ad) == n && aligned16(ad->data) &&
           ((ad->src[0] == a && ad->src[1] == b) || (ad->src[0] == b && ad->src[1] == a));
}

bool match_persist_layer(ggml_cgraph *g, int i, const Consumers &C, PersistLayerMatch &P) {
    const int nn = ggml_graph_n_nodes(g);
    AttnInMatch M;
    if (!match_attn_in(g, i, C, M) || M.wt != GGML_TYPE_Q8_0) return false;
    const ggml_tensor *const *mm = M.mm;
    P.x = M.x;
    P.rms = ggml_graph_node(g, i);
    P.hd = M.hd;
    P.n_embd = M.x->ne[0];
    P.n_head = mm[0]->ne[0] / M.hd;
    P.n_head_kv = mm[1]->ne[0] / M.hd;
    P.eps = M.eps;
    P.rope = M.rope[0];
    P.idx = M.sr[0]->src[1];
    if (mm[1]->ne[0] != mm[2]->ne[0] || !aligned16(M.nw->data)) return false;
    // attention: one sequence, one query row, over the caches just written; the mask, if
    // any, is one F16 row (supports_fa: >= n_kv elements, shared by the heads)
    int j = next_real(g, M.end + 1);
    if (j >= nn) return false;
    const ggml_tensor *fa = ggml_graph_node(g, j);
    if (fa->op != GGML_OP_FLASH_ATTN_EXT || !supports_fa(fa)) return false;
    const ggml_tensor *q = fa->src[0], *k = fa->src[1], *v = fa->src[2], *mask = fa->src[3];
    if ((mask && mask->ne[3] != 1) || q->data != M.rope[0]->data || q->ne[0] != P.hd || q->ne[1] != 1 || q->ne[2] != P.n_head ||
        q->ne[3] != 1 || k->ne[2] != P.n_head_kv || k->ne[3] != 1 || k->data != M.sr[0]->data ||
        v->data != M.sr[1]->data || k->nb[1] != M.sr[0]->nb[1] || v->nb[1] != M.sr[1]->nb[1] || v->nb[1] != k->nb[1] ||
        k->nb[2] != (size_t)P.hd * 2 || v->nb[2] != (size_t)P.hd * 2 || !only_consumed_by(C, M.rope[0], {fa}) ||
        !aligned16(k->data) || !aligned16(v->data))
        return false;
    P.fa = fa;
    P.mask = mask ? mask->data : nullptr;
    P.kvl = fa->src[5];
    P.n_kv = k->ne[1];
    P.kv_row_bytes = k->nb[1];
    P.n_cache_rows = std::min(M.sr[0]->ne[1], M.sr[1]->ne[1]);
    memcpy(&P.kq_scale, fa->op_params, sizeof(float));
    // o projection + residual
    j = next_real(g, j + 1);
    if (j >= nn) return false;
    const ggml_tensor *mo = ggml_graph_node(g, j);
    if (!q8_gemv_node(mo) || alias_root(mo->src[1]) != fa || !only_consumed_by(C, fa, {mo}) ||
        mo->src[0]->ne[0] != P.n_head * P.hd || mo->src[0]->ne[1] != P.n_embd)
        return false;
    j = next_real(g, j + 1);
    if (j >= nn) return false;
    const ggml_tensor *x1 = ggml_graph_node(g, j);
    if (!is_add_of(x1, mo, M.x, P.n_embd) || !only_consumed_by(C, mo, {x1})) return false;
    // FFN
    j = next_real(g, j + 1);
    if (j >= nn) return false;
    const ggml_tensor *x2, *nw2, *mul2;
    const int j_rms = j;
    if (!rms_mul_head(g, j_rms, C, j, x2, nw2, mul2, P.eps_ffn) || x2 != x1 || !aligned16(nw2->data)) return false;
    const ggml_tensor *gu[2];
    for (int t = 0; t < 2; t++) {
        j = next_real(g, j + 1);
        if (j >= nn) return false;
        gu[t] = ggml_graph_node(g, j);
        if (!q8_gemv_node(gu[t]) || gu[t]->src[1] != mul2 || gu[t]->src[0]->ne[0] != P.n_embd ||
            inv_s_of(gu[t]->src[0]) != inv_s_of(gu[0]->src[0]))
            return false;
    }
    P.n_ff = gu[0]->ne[0];
    if (gu[1]->ne[0] != P.n_ff || !only_consumed_by(C, mul2, {gu[0], gu[1]})) return false;
    j = next_real(g, j + 1);
    if (j >= nn) return false;
    const ggml_tensor *glu = ggml_graph_node(g, j);
    if (glu->op != GGML_OP_GLU || !supports_op_impl(glu) || glu->src[0] != gu[0] || glu->src[1] != gu[1] ||
        !only_consumed_by(C, gu[0], {glu}) || !only_consumed_by(C, gu[1], {glu}))
        return false;
    j = next_real(g, j + 1);
    if (j >= nn) return false;
    const ggml_tensor *down = ggml_graph_node(g, j);
    if (!q8_gemv_node(down) || down->src[1] != glu || !only_consumed_by(C, glu, {down}) ||
        down->src[0]->ne[0] != P.n_ff || down->src[0]->ne[1] != P.n_embd)
        return false;
    j = next_real(g, j + 1);
    if (j >= nn) return false;
    const ggml_tensor *out = ggml_graph_node(g, j);
    if (!is_add_of(out, down, x1, P.n_embd) || !only_consumed_by(C, down, {out}) ||
        !only_consumed_by(C, x1, {ggml_graph_node(g, j_rms), out}))
        return false;
    P.out = out;
    P.x1 = x1;
    P.end = j;
    mi_persist_layer &L = P.L;
    auto packed = [](const ggml_tensor *mmn) { return ((const TensorExtra *)mmn->src[0]->extra)->packed; };
    L.wq = packed(mm[0]);
    L.wk = packed(mm[1]);
    L.wv = packed(mm[2]);
    L.wo = packed(mo);
    L.w_gate = packed(gu[0]);
    L.w_up = packed(gu[1]);
    L.w_down = packed(down);
    L.bq = M.bias[0] ? (const float *)M.bias[0]->data : nullptr;
    L.bk = M.bias[1] ? (const float *)M.bias[1]->data : nullptr;
    L.bv = M.bias[2] ? (const float *)M.bias[2]->data : nullptr;
    L.attn_norm = (const float *)M.nw->data;
    L.ffn_norm = (const float *)nw2->data;
    L.inv_s_attn = inv_s_of(mm[0]->src[0]);
    L.inv_s_o = inv_s_of(mo->src[0]);
    L.inv_s_ffn = inv_s_of(gu[0]->src[0]);
    L.inv_s_down = inv_s_of(down->src[0]);
    L.k_cache = M.sr[0]->data;
    L.v_cache = M.sr[1]->data;
    return true;
}

// the values one launch shares over its layers
bool persist_same_step(const PersistLayerMatch &a, const PersistLayerMatch &b) {
    float fa0[3], fb0[3];
    rope_params(a.rope, fa0[0], fa0[1], fa0[2]);
    rope_params(b.rope, fb0[0], fb0[1], fb0[2]);
    return a.rope->src[1] == b.rope->src[1] && a.idx == b.idx && a.kvl == b.kvl && a.mask == b.mask &&
           a.eps == b.eps &&
           a.eps_ffn == b.eps && b.eps_ffn == b.eps && a.kq_scale == b.kq_scale && a.n_embd == b.n_embd &&
           a.n_head == b.n_head && a.n_head_kv == b.n_head_kv && a.hd == b.hd && a.n_ff == b.n_ff &&
           a.n_kv == b.n_kv && a.n_cache_rows == b.n_cache_rows && a.kv_row_bytes == b.kv_row_bytes &&
           memcmp(fa0, fb0, sizeof(fa0)) == 0 && a.idx->type == b.idx->type;
}

// folds the last timed persistent launch into the totals (waits for its end event)
void collect_persist_timing(BackendCtx *ctx) {
    if (!ctx->pt_pending) return;
    float ms = 0.0f;
    MI_HIP_CHECK(hipEventSynchronize(ctx->pt_ev[1]));
    MI_HIP_CHECK(hipEventElapsedTime(&ms, ctx->pt_ev[0], ctx->pt_ev[1]));
    ctx->pt_ms += ms;
    ctx->pt_launches++;
    ctx->pt_pending = false;
}

// embd_rows: the GET_ROWS node whose output is the run's input (try_fuse_persist_embd)
int try_fuse_persist(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C,
                     const ggml_tensor *embd_rows = nullptr) {
    if (!ctx->persist_on || ctx->persist_failed) return 0;
    std::vector<PersistLayerMatch> run;
    PersistLayerMatch P;
    for (int at = i; match_persist_layer(g, at, C, P); at = next_real(g, P.end + 1)) {
        // the layer outputs inside the run are never written: only the next layer may read them
        if (!run.empty() && (P.x != run.back().out || !persist_same_step(run.front(), P) ||
                             !only_consumed_by(C, P.x, {P.rms, P.x1})))
            break;
        if (run.empty() && P.eps_ffn != P.eps) return 0;
        run.push_back(P);
        if (next_real(g, P.end + 1) >= ggml_graph_n_nodes(g)) break;
    }
    if (run.empty()) return 0;
    const PersistLayerMatch &F = run.front();
    if (embd_rows && (F.x != embd_rows || !only_consumed_by(C, embd_rows, {F.rms, F.x1}))) return 0;
    if (!mi_persist_supported(F.n_kv, (int)F.n_embd, (int)F.n_head, (int)F.n_head_kv, (int)F.hd, (int)F.n_ff))
        return 0;
    const int n_layer = (int)run.size();
    if (!ctx->persist || ctx->persist_layers != n_layer) {
        if (ctx->persist) {
            MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
            mi_persist_destroy(ctx->persist);
            ctx->persist = nullptr;
        }
        if (mi_persist_create(&ctx->persist, ctx->device, n_layer, (int)F.n_embd, (int)F.n_head, (int)F.n_head_kv,
                              (int)F.hd, (int)F.n_ff) != MI_OK) {
            fprintf(stderr, "MI355X: persistent decode unavailable (%s); per-node path\n", mi_last_error());
            ctx->persist = nullptr;
            ctx->persist_failed = true;
            return 0;
        }
        ctx->persist_layers = n_layer;
        if (!ctx->persist_trace.empty()) MI_K_CHECK(mi_persist_enable_trace(ctx->persist));
    }
    std::vector<mi_persist_layer> layers(n_layer);
    for (int l = 0; l < n_layer; l++) layers[l] = run[l].L;
    MI_K_CHECK(mi_persist_set_layers(ctx->stream, ctx->persist, layers.data(), n_layer));
    mi_persist_args a{};
    if (embd_rows) {  // the run reads the token's embedding row itself (GET_ROWS not launched)
        a.x_in = nullptr;
        a.embd = (const uint16_t *)embd_rows->src[0]->data;
        a.embd_ld = (int64_t)(embd_rows->src[0]->nb[1] / 2);
        a.tok = (const int32_t *)embd_rows->src[1]->data;
    } else {
        a.x_in = (const float *)F.x->data;
    }
    a.x_out = (float *)run.back().out->data;
    a.pos = (const int32_t *)F.rope->src[1]->data;
    a.kv_idx = F.idx->data;
    a.kv_idx_is_i64 = F.idx->type == GGML_TYPE_I64;
    a.n_cache_rows = F.n_cache_rows;
    a.kv_row_bytes = F.kv_row_bytes;
    a.n_kv = (int)F.n_kv;
    a.kv_len = F.kvl ? (const int32_t *)F.kvl->data : nullptr;
    a.mask = (const uint16_t *)F.mask;
    a.kq_scale = F.kq_scale;
    a.rms_eps = F.eps;
    rope_params(F.rope, a.freq_base, a.freq_scale, a.attn_factor);
    a.rounding = q8_rounding();
    // test hooks, read per call: a short bounded wait and a hop that never completes
    const char *spin = getenv("GGML_MI355X_PERSIST_SPIN"), *stall = getenv("GGML_MI355X_PERSIST_STALL_HOP");
    a.spin_limit = spin && *spin ? atol(spin) : 0;
    a.debug_stall_hop = stall && *stall ? atoi(stall) : -1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    MI_HIP_CHECK(hipStreamIsCapturing(ctx->stream, &cap));
    const bool timed = ctx->persist_timing && cap == hipStreamCaptureStatusNone;
    if (timed) {
        collect_persist_timing(ctx);  // one event pair: a launch not yet read is read first
        MI_HIP_CHECK(hipEventRecord(ctx->pt_ev[0], ctx->stream));
    }
    MI_K_CHECK(mi_persist_decode_q8_0(ctx->stream, ctx->persist, &a));
    if (timed) {
        MI_HIP_CHECK(hipEventRecord(ctx->pt_ev[1], ctx->stream));
        ctx->pt_pending = true;
    }
    return run.back().end + 1 - i;
}

// GET_ROWS (one token's F16 embedding row) read only by the first layer of a persistent
// run that follows it: the run reads the row itself, so the GET_ROWS launch and its fp32
// row go
int try_fuse_persist_embd(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    if (!ctx->persist_on || ctx->persist_failed) return 0;
    const ggml_tensor *gr = ggml_graph_node(g, i);
    const ggml_tensor *t = gr->src[0], *ids = gr->src[1];
    if (t->type != GGML_TYPE_F16 || ids->type != GGML_TYPE_I32 || ggml_nelements(ids) != 1 ||
        gr->type != GGML_TYPE_F32 || ggml_nrows(gr) != 1 || t->ne[0] != gr->ne[0] || t->nb[0] != 2 || t->nb[1] % 8 ||
        ((uintptr_t)t->data & 7))
        return 0;
    const int j = next_real(g, i + 1);
    if (j >= ggml_graph_n_nodes(g) || ggml_graph_node(g, j)->op != GGML_OP_RMS_NORM) return 0;
    const int used = try_fuse_persist(ctx, g, j, C, gr);
    return used ? j + used - i : 0;
}

// ---- several activation rows (a ubatch of tokens) through Q4_0 weights

// a Q4_0 MUL_MAT on 2..16 contiguous fp32 activation rows with the prepacked copy ready
bool q4_batch_node(const ggml_tensor *n) {
    if (n->op != GGML_OP_MUL_MAT) return false;
    const ggml_tensor *a = n->src[0], *b = n->src[1];
    const TensorExtra *ex = (const TensorExtra *)a->extra;
    const int64_t m = ggml_nrows(b);
    return a->type == GGML_TYPE_Q4_0 && ex && ex->ready && b->type == GGML_TYPE_F32 && ggml_is_contiguous(b) &&
           b->ne[1] == m && m >= 2 && m <= 16 && a->ne[0] % 128 == 0 && is_f32_contig(n);
}

// a Q8_0 MUL_MAT on 2..8 contiguous fp32 activation rows with the prepacked copy ready
bool q8_batch_node(const ggml_tensor *n) {
    if (n->op != GGML_OP_MUL_MAT) return false;
    const ggml_tensor *a = n->src[0], *b = n->src[1];
    const TensorExtra *ex = (const TensorExtra *)a->extra;
    const int64_t m = ggml_nrows(b);
    return packed_fmt(a) == GGML_TYPE_Q8_0 && ex && ex->ready && b->type == GGML_TYPE_F32 && ggml_is_contiguous(b) &&
           b->ne[1] == m && m >= 2 && m <= 8 && a->ne[0] % 32 == 0 && aligned16(b->data) && is_f32_contig(n);
}

// ADD(mm, other) as mm's only consumer: other is a bias row of mm's width (broadcast over
// the rows) or a tensor of mm's shape (the residual)
const ggml_tensor *batch_add_tail(ggml_cgraph *g, int j, const ggml_tensor *mm, const Consumers &C,
                                  const ggml_tensor *&other, bool &is_bias) {
    const int k = next_real(g, j + 1);
    if (k >= ggml_graph_n_nodes(g)) return nullptr;
    const ggml_tensor *ad = ggml_graph_node(g, k);
    if (ad->op != GGML_OP_ADD || ad->src[0] != mm || !is_f32_contig(ad) || !ggml_are_same_shape(ad, mm)) return nullptr;
    const ggml_tensor *o = ad->src[1];
    if (!is_f32_contig(o) || o == mm || !only_consumed_by(C, mm, {ad})) return nullptr;
    if (ggml_nelements(o) == mm->ne[0] && o->ne[0] == mm->ne[0]) is_bias = true;
    else if (ggml_are_same_shape(o, mm)) is_bias = false;
    else return nullptr;
    other = o;
    return ad;
}

// MUL_MAT x 1..4 (Q4_0, same activation rows) [-> ADD bias per matrix, in order] or
// MUL_MAT -> ADD(residual): one conversion of the activation, one launch.  The group
// starts at node i0; with norm (RMS_NORM -> MUL(norm_w) at node i, the MUL being the
// matmuls' activation and read by nothing else) the norm runs in the conversion.
struct BatchNorm {
    const ggml_tensor *x = nullptr, *w = nullptr;
    float eps = 0.0f;
};

// gate, up (the group just matched) -> GLU swiglu -> down MUL_MAT [-> ADD]: gate and up
// form the swiglu in their epilogue, written as the down projection's permuted fp16
// activation (no gate/up outputs, no GLU tensor, no conversion launch)
int fuse_q4_glu_pair(BackendCtx *ctx, ggml_cgraph *g, int i, int last, const Consumers &C,
                     const ggml_tensor *const *mm, const float *x, const BatchNorm &norm, int64_t k, int64_t m) {
    const int nn = ggml_graph_n_nodes(g);
    const int64_t n = mm[0]->src[0]->ne[1];
    if (mm[1]->src[0]->ne[1] != n || n % 128) return 0;
    const int jg = next_real(g, last + 1);
    if (jg >= nn) return 0;
    const ggml_tensor *glu = ggml_graph_node(g, jg);
    if (glu->op != GGML_OP_GLU || !supports_op_impl(glu) || glu->src[0] != mm[0] || glu->src[1] != mm[1] ||
        !only_consumed_by(C, mm[0], {glu}) || !only_consumed_by(C, mm[1], {glu}))
        return 0;
    const int jd = next_real(g, jg + 1);
    if (jd >= nn) return 0;
    const ggml_tensor *down = ggml_graph_node(g, jd);
    if (!q4_batch_node(down) || down->src[1] != glu || !only_consumed_by(C, glu, {down}) ||
        down->src[0]->ne[0] != n)
        return 0;
    const size_t need_in = ((size_t)(m * k * 2) + 255) / 256 * 256, need_h = (size_t)(m * n * 2);
    if (need_in + need_h > ctx->scratch_size) return 0;
    const ggml_tensor *other = nullptr;
    bool is_bias = false;
    const ggml_tensor *ad = batch_add_tail(g, jd, down, C, other, is_bias);
    uint8_t *hxp = (uint8_t *)ctx->scratch + need_in;
    MI_K_CHECK(mi_mul_mat_q4_0_gate_up_glu_batch(ctx->stream, ((const TensorExtra *)mm[0]->src[0]->extra)->packed,
                                                 ((const TensorExtra *)mm[1]->src[0]->extra)->packed, n, k, m, x,
                                                 norm.w ? (const float *)norm.w->data : nullptr, norm.eps,
                                                 ctx->scratch, need_in, hxp));
    const void *w = ((const TensorExtra *)down->src[0]->extra)->packed;
    const int64_t nd = down->src[0]->ne[1];
    float *y = (float *)(ad ? ad->data : down->data);
    const float *bv = ad && is_bias ? (const float *)other->data : nullptr;
    const float *av = ad && !is_bias ? (const float *)other->data : nullptr;
    MI_K_CHECK(mi_mul_mat_q4_0_batch_xp(ctx->stream, 1, &w, &nd, &y, &bv, &av, n, m, hxp));
    return (ad ? next_real(g, jd + 1) : jd) + 1 - i;
}

struct RopeKvMatch;
bool match_rope_kv(ggml_cgraph *g, int i, const Consumers &C, RopeKvMatch &R);
int fuse_q4_qkv_rope(BackendCtx *ctx, ggml_cgraph *g, int i, int tail, const Consumers &C,
                     const ggml_tensor *const *mm, const ggml_tensor *const *ad, const ggml_tensor *const *bias,
                     const float *x, const BatchNorm &norm, int64_t k, int64_t m);

int fuse_q4_batch_at(BackendCtx *ctx, ggml_cgraph *g, int i, int i0, const Consumers &C, const BatchNorm &norm) {
    const int nn = ggml_graph_n_nodes(g);
    ggml_tensor *mm0 = ggml_graph_node(g, i0);
    if (!q4_batch_node(mm0)) return 0;
    const ggml_tensor *mm[4] = {mm0};
    int cnt = 1, last = i0;
    while (cnt < 4) {
        const int j = next_real(g, last + 1);
        if (j >= nn) break;
        const ggml_tensor *nx = ggml_graph_node(g, j);
        if (!q4_batch_node(nx) || nx->src[1] != mm0->src[1] || nx->src[0]->ne[0] != mm0->src[0]->ne[0]) break;
        mm[cnt++] = nx;
        last = j;
    }
    // the ADD of each matrix's output, adjacent after the group in matrix order
    const ggml_tensor *ad[4] = {}, *other[4] = {};
    bool bias[4] = {};
    int tail = last;
    bool all_add = true;
    for (int t = 0; t < cnt && all_add; t++) {
        const ggml_tensor *a = batch_add_tail(g, tail, mm[t], C, other[t], bias[t]);
        if (!a || (cnt > 1 && !bias[t])) all_add = false;
        ad[t] = a;
        if (a) tail = next_real(g, tail + 1);
    }
    if (!all_add) tail = last;
    if (cnt == 1 && !all_add && !norm.w) return 0;  // a lone matmul takes the plain path
    if (norm.w) {
        std::vector<const ggml_tensor *> cs;
        real_consumers(C, mm0->src[1], cs);
        if (cs.size() != (size_t)cnt) return 0;  // the normed activation is read only by the group
        for (const ggml_tensor *c : cs)
            if (std::find(mm, mm + cnt, c) == mm + cnt) return 0;
    }
    const void *w[4];
    int64_t n[4];
    float *y[4];
    const float *bv[4], *av[4];
    for (int t = 0; t < cnt; t++) {
        w[t] = ((const TensorExtra *)mm[t]->src[0]->extra)->packed;
        n[t] = mm[t]->src[0]->ne[1];
        y[t] = (float *)(all_add ? ad[t]->data : mm[t]->data);
        bv[t] = all_add && bias[t] ? (const float *)other[t]->data : nullptr;
        av[t] = all_add && !bias[t] ? (const float *)other[t]->data : nullptr;
    }
    const int64_t k = mm0->src[0]->ne[0], m = ggml_nrows(mm0->src[1]);
    const float *x = (const float *)(norm.w ? norm.x->data : mm0->src[1]->data);
    if (cnt == 2 && !all_add) {
        if (int used = fuse_q4_glu_pair(ctx, g, i, last, C, mm, x, norm, k, m)) return used;
    }
    if (cnt == 3 && all_add && bias[0] && bias[1] && bias[2]) {
        if (int used = fuse_q4_qkv_rope(ctx, g, i, tail, C, mm, ad, other, x, norm, k, m)) return used;
    }
    MI_K_CHECK(mi_mul_mat_q4_0_f32_batch(ctx->stream, cnt, w, n, y, bv, av, k, m, x, nullptr,
                                         norm.w ? (const float *)norm.w->data : nullptr, norm.eps, ctx->scratch,
                                         ctx->scratch_size));
    return tail + 1 - i;
}

int try_fuse_q4_batch(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    return fuse_q4_batch_at(ctx, g, i, i, C, BatchNorm{});
}

// MUL_MAT x 1..4 (Q8_0, the same 2..8 activation rows and SmoothQuant divisors)
// [-> ADD bias per matrix, in order] or MUL_MAT -> ADD(residual), starting at node i0,
// optionally after RMS_NORM -> MUL(norm_w) at node i: one quantization of the activation
// rows (norm folded in) and one launch over the stacked matrices.
int fuse_q8_batch_at(BackendCtx *ctx, ggml_cgraph *g, int i, int i0, const Consumers &C, const BatchNorm &norm) {
    const int nn = ggml_graph_n_nodes(g);
    ggml_tensor *mm0 = ggml_graph_node(g, i0);
    if (!q8_batch_node(mm0)) return 0;
    const ggml_tensor *mm[4] = {mm0};
    int cnt = 1, last = i0;
    while (cnt < 4) {
        const int j = next_real(g, last + 1);
        if (j >= nn) break;
        const ggml_tensor *nx = ggml_graph_node(g, j);
        if (!q8_batch_node(nx) || nx->src[1] != mm0->src[1] || nx->src[0]->ne[0] != mm0->src[0]->ne[0] ||
            inv_s_of(nx->src[0]) != inv_s_of(mm0->src[0]))
            break;
        mm[cnt++] = nx;
        last = j;
    }
    const ggml_tensor *ad[4] = {}, *other[4] = {};
    bool bias[4] = {};
    int tail = last;
    bool all_add = true;
    for (int t = 0; t < cnt && all_add; t++) {
        const ggml_tensor *a = batch_add_tail(g, tail, mm[t], C, other[t], bias[t]);
        if (!a || (cnt > 1 && !bias[t])) all_add = false;
        ad[t] = a;
        if (a) tail = next_real(g, tail + 1);
    }
    if (!all_add) tail = last;
    if (norm.w) {
        std::vector<const ggml_tensor *> cs;
        real_consumers(C, mm0->src[1], cs);
        if (cs.size() != (size_t)cnt) return 0;  // the normed activation is read only by the group
        for (const ggml_tensor *c : cs)
            if (std::find(mm, mm + cnt, c) == mm + cnt) return 0;
    }
    const int64_t k = mm0->src[0]->ne[0], m = ggml_nrows(mm0->src[1]);
    if (norm.w && k > 4096) return 0;
    if (ctx->scratch_size < mi_xq_size(m, k)) return 0;
    const void *w[4];
    int64_t n[4];
    float *y[4];
    const float *bv[4], *av[4];
    for (int t = 0; t < cnt; t++) {
        w[t] = ((const TensorExtra *)mm[t]->src[0]->extra)->packed;
        n[t] = mm[t]->src[0]->ne[1];
        y[t] = (float *)(all_add ? ad[t]->data : mm[t]->data);
        bv[t] = all_add && bias[t] ? (const float *)other[t]->data : nullptr;
        av[t] = all_add && !bias[t] ? (const float *)other[t]->data : nullptr;
    }
    const float *x = (const float *)(norm.w ? norm.x->data : mm0->src[1]->data);
    MI_K_CHECK(mi_mul_mat_q8_0_f32_batch(ctx->stream, cnt, w, n, y, bv, av, k, m, x, nullptr,
                                         norm.w ? (const float *)norm.w->data : nullptr, norm.eps,
                                         inv_s_of(mm0->src[0]), q8_rounding(), ctx->scratch, ctx->scratch_size));
    return tail + 1 - i;
}

int try_fuse_q8_batch(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    return fuse_q8_batch_at(ctx, g, i, i, C, BatchNorm{});
}

// FLASH_ATTN_EXT (several sequences, one token each) whose output only feeds a Q4_0
// projection of those rows [-> ADD bias or residual]: the attention's combine writes the
// projection's permuted fp16 activation straight into the scratch (no attention-output
// tensor, no conversion launch), then the matrix-core projection reads it.
int try_fuse_fa_q4_batch(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    const ggml_tensor *fa = ggml_graph_node(g, i);
    const ggml_tensor *q = fa->src[0], *k = fa->src[1], *v = fa->src[2], *mask = fa->src[3];
    const ggml_tensor *kvl = fa->src[5];
    const int64_t n_seq = q->ne[3], d = q->ne[0], n_head = q->ne[2];
    if (n_seq < 2 || q->ne[1] != 1 || !ggml_is_contiguous(fa)) return 0;
    const int j = next_real(g, i + 1);
    if (j >= ggml_graph_n_nodes(g)) return 0;
    const ggml_tensor *mm = ggml_graph_node(g, j);
    if (!q4_batch_node(mm) || alias_root(mm->src[1]) != fa || !only_consumed_by(C, fa, {mm})) return 0;
    const int64_t kk = mm->src[0]->ne[0], m = ggml_nrows(mm->src[1]);
    if (kk != d * n_head || m != n_seq || (size_t)(m * kk * 2) > ctx->scratch_size) return 0;
    const ggml_tensor *other = nullptr;
    bool is_bias = false;
    const ggml_tensor *ad = batch_add_tail(g, j, mm, C, other, is_bias);
    float scale;
    memcpy(&scale, fa->op_params, sizeof(float));
    const size_t mask_seq = mask && mask->ne[3] > 1 ? mask->nb[3] / 2 : 0;
    MI_K_CHECK(mi_fa_decode_batch_q4act(ctx->stream, (const float *)q->data, k->data, v->data,
                                        mask ? (const uint16_t *)mask->data : nullptr,
                                        kvl ? (const int32_t *)kvl->data : nullptr, k->ne[1], n_head, k->ne[2], d,
                                        k->nb[1], k->nb[2], v->nb[1], v->nb[2], scale, ctx->scratch, n_seq,
                                        q->nb[3] / 4, k->nb[3], v->nb[3], mask_seq, ctx->fa_ws, ctx->fa_ws_size));
    const void *w = ((const TensorExtra *)mm->src[0]->extra)->packed;
    const int64_t n = mm->src[0]->ne[1];
    float *y = (float *)(ad ? ad->data : mm->data);
    const float *bv = ad && is_bias ? (const float *)other->data : nullptr;
    const float *av = ad && !is_bias ? (const float *)other->data : nullptr;
    MI_K_CHECK(mi_mul_mat_q4_0_batch_xp(ctx->stream, 1, &w, &n, &y, &bv, &av, kk, m, ctx->scratch));
    return (ad ? next_real(g, j + 1) : j) + 1 - i;
}

// RMS_NORM (2..16 rows, k <= 4096) -> MUL(norm_w row) -> the Q4_0 group of try_fuse_q4_batch
int try_fuse_norm_q4_batch(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    const int nn = ggml_graph_n_nodes(g);
    const ggml_tensor *rms = ggml_graph_node(g, i);
    const ggml_tensor *x = rms->src[0];
    const int64_t m = ggml_nrows(x);
    if (!is_f32_contig(x) || m < 2 || m > 16 || x->ne[1] != m || x->ne[0] > 4096 || x->ne[0] % 32 ||
        !aligned16(x->data))
        return 0;
    const int j = next_real(g, i + 1);
    if (j >= nn) return 0;
    const ggml_tensor *mul = ggml_graph_node(g, j);
    if (mul->op != GGML_OP_MUL || mul->src[0] != rms || !is_row_vector(mul->src[1], x->ne[0]) ||
        !only_consumed_by(C, rms, {mul}))
        return 0;
    const int i0 = next_real(g, j + 1);
    if (i0 >= nn || ggml_graph_node(g, i0)->src[1] != mul) return 0;
    BatchNorm norm;
    norm.x = x;
    norm.w = mul->src[1];
    memcpy(&norm.eps, rms->op_params, sizeof(float));
    if (!aligned16(norm.w->data)) return 0;
    if (q8_batch_node(ggml_graph_node(g, i0))) return fuse_q8_batch_at(ctx, g, i, i0, C, norm);
    if (x->ne[0] % 128) return 0;
    return fuse_q4_batch_at(ctx, g, i, i0, C, norm);
}

// GLU swiglu (gate, up: 2..16 rows) -> MUL_MAT(Q4_0) [-> ADD residual]: the swiglu is
// formed while the activation is converted for the matrix cores
int try_fuse_glu_q4_batch(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    const ggml_tensor *glu = ggml_graph_node(g, i);
    if (glu->op != GGML_OP_GLU || !supports_op_impl(glu) || !glu->src[1] || !is_f32_contig(glu->src[0]) ||
        !is_f32_contig(glu->src[1]) || !ggml_are_same_shape(glu->src[0], glu->src[1]))
        return 0;
    const int j = next_real(g, i + 1);
    if (j >= ggml_graph_n_nodes(g)) return 0;
    const ggml_tensor *mm = ggml_graph_node(g, j);
    const bool q8 = q8_batch_node(mm);
    if ((!q8 && !q4_batch_node(mm)) || mm->src[1] != glu || !only_consumed_by(C, glu, {mm})) return 0;
    const ggml_tensor *other = nullptr;
    bool is_bias = false;
    const ggml_tensor *ad = batch_add_tail(g, j, mm, C, other, is_bias);
    const void *w = ((const TensorExtra *)mm->src[0]->extra)->packed;
    const int64_t n = mm->src[0]->ne[1], k = mm->src[0]->ne[0], m = ggml_nrows(glu);
    float *y = (float *)(ad ? ad->data : mm->data);
    const float *bv = ad && is_bias ? (const float *)other->data : nullptr;
    const float *av = ad && !is_bias ? (const float *)other->data : nullptr;
    if (q8) {  // the swiglu formed while the down projection's activation rows are quantized
        if (!aligned16(glu->src[0]->data) || !aligned16(glu->src[1]->data) || ctx->scratch_size < mi_xq_size(m, k))
            return 0;
        MI_K_CHECK(mi_mul_mat_q8_0_f32_batch(ctx->stream, 1, &w, &n, &y, &bv, &av, k, m,
                                             (const float *)glu->src[0]->data, (const float *)glu->src[1]->data,
                                             nullptr, 0.0f, inv_s_of(mm->src[0]), q8_rounding(), ctx->scratch,
                                             ctx->scratch_size));
        return (ad ? next_real(g, j + 1) : j) + 1 - i;
    }
    MI_K_CHECK(mi_mul_mat_q4_0_f32_batch(ctx->stream, 1, &w, &n, &y, &bv, &av, k, m, (const float *)glu->src[0]->data,
                                         (const float *)glu->src[1]->data, nullptr, 0.0f, ctx->scratch,
                                         ctx->scratch_size));
    return (ad ? next_real(g, j + 1) : j) + 1 - i;
}

// ROPE q, ROPE k (same positions and parameters, all head dims rotated), SET_ROWS of the
// rotated k, SET_ROWS of v (same row indices): one launch over the ubatch's rows
// ROPE q, ROPE k, SET_ROWS k, SET_ROWS v starting at node i (views between them skipped)
struct RopeKvMatch {
    const ggml_tensor *rope[2], *sr[2], *v, *pos, *idx;
    int64_t hd, m;
    float freq_base, freq_scale, attn_factor;
    int last;  // the last node of the run
};

bool match_rope_kv(ggml_cgraph *g, int i, const Consumers &C, RopeKvMatch &R) {
    const int nn = ggml_graph_n_nodes(g);
    int j = i;
    for (int t = 0; t < 2; t++) {
        if (t) j = next_real(g, j + 1);
        if (j >= nn) return false;
        R.rope[t] = ggml_graph_node(g, j);
        const ggml_tensor *x = R.rope[t]->src[0];
        if (R.rope[t]->op != GGML_OP_ROPE || !supports_op_impl(R.rope[t]) || !is_f32_contig(x) ||
            !is_f32_contig(R.rope[t]) || R.rope[t]->op_params[1] != x->ne[0] || x->ne[3] != 1)
            return false;
    }
    R.hd = R.rope[0]->src[0]->ne[0];
    R.m = R.rope[0]->src[0]->ne[2];
    R.pos = R.rope[0]->src[1];
    if (R.rope[1]->src[0]->ne[0] != R.hd || R.rope[1]->src[0]->ne[2] != R.m || R.rope[1]->src[1] != R.pos ||
        ggml_nelements(R.pos) != R.m || R.hd > 256 ||
        memcmp(R.rope[0]->op_params + 5, R.rope[1]->op_params + 5, 4 * sizeof(int32_t)) != 0)
        return false;
    for (int t = 0; t < 2; t++) {
        j = next_real(g, j + 1);
        if (j >= nn) return false;
        R.sr[t] = ggml_graph_node(g, j);
        const ggml_tensor *src = R.sr[t]->src[0];
        if (R.sr[t]->op != GGML_OP_SET_ROWS || !supports_op_impl(R.sr[t]) || !is_f32_contig(src) ||
            ggml_nrows(src) != R.m || ggml_nelements(R.sr[t]->src[1]) != R.m ||
            (t == 1 && R.sr[1]->src[1] != R.sr[0]->src[1]))
            return false;
    }
    if (alias_root(R.sr[0]->src[0]) != R.rope[1] || R.sr[0]->src[0]->ne[0] != R.rope[1]->src[0]->ne[1] * R.hd ||
        !only_consumed_by(C, R.rope[1], {R.sr[0]}))
        return false;
    R.v = R.sr[1]->src[0];
    R.idx = R.sr[0]->src[1];
    memcpy(&R.freq_base, (const float *)R.rope[0]->op_params + 5, sizeof(float));
    memcpy(&R.freq_scale, (const float *)R.rope[0]->op_params + 6, sizeof(float));
    memcpy(&R.attn_factor, (const float *)R.rope[0]->op_params + 8, sizeof(float));
    R.last = j;
    return true;
}

int try_fuse_rope_kv(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    RopeKvMatch R;
    if (!match_rope_kv(g, i, C, R)) return 0;
    // q_out is written while other workgroups read k and v
    if (overlaps(R.rope[0], alias_root(R.rope[1]->src[0])) || overlaps(R.rope[0], R.v)) return 0;
    MI_K_CHECK(mi_rope_kv_rows(ctx->stream, (const float *)R.rope[0]->src[0]->data,
                               (const float *)R.rope[1]->src[0]->data, (const float *)R.v->data,
                               (float *)R.rope[0]->data, R.sr[0]->data, R.sr[0]->nb[1], R.sr[1]->data, R.sr[1]->nb[1],
                               (const int32_t *)R.pos->data, R.idx->data, R.idx->type == GGML_TYPE_I64,
                               std::min(R.sr[0]->ne[1], R.sr[1]->ne[1]), R.m, R.hd, R.rope[0]->src[0]->ne[1],
                               R.rope[1]->src[0]->ne[1], R.v->ne[0], R.freq_base, R.freq_scale, R.attn_factor));
    return R.last + 1 - i;
}

// q, k, v (+ bias each: the group just matched) -> ROPE q, ROPE k, SET_ROWS k, SET_ROWS v:
// the rotation and the cache writes run in the projection's epilogue (PAIR_ROPE), so
// neither the projected rows nor the rotated k are written to memory
int fuse_q4_qkv_rope(BackendCtx *ctx, ggml_cgraph *g, int i, int tail, const Consumers &C,
                     const ggml_tensor *const *mm, const ggml_tensor *const *ad, const ggml_tensor *const *bias,
                     const float *x, const BatchNorm &norm, int64_t k, int64_t m) {
    const int ir = next_real(g, tail + 1);
    if (ir >= ggml_graph_n_nodes(g)) return 0;
    RopeKvMatch R;
    if (!match_rope_kv(g, ir, C, R)) return 0;
    if (R.m != m || alias_root(R.rope[0]->src[0]) != ad[0] || alias_root(R.rope[1]->src[0]) != ad[1] ||
        alias_root(R.v) != ad[2] || !only_consumed_by(C, ad[0], {R.rope[0]}) ||
        !only_consumed_by(C, ad[1], {R.rope[1]}) || !only_consumed_by(C, ad[2], {R.sr[1]}))
        return 0;
    const int64_t n[3] = {mm[0]->src[0]->ne[1], mm[1]->src[0]->ne[1], mm[2]->src[0]->ne[1]};
    if (R.hd % 32 || n[0] % R.hd || n[1] % R.hd || n[2] % 32 || R.rope[0]->src[0]->ne[1] * R.hd != n[0] ||
        R.rope[1]->src[0]->ne[1] * R.hd != n[1] || R.v->ne[0] != n[2] || ctx->scratch_size < (size_t)(m * k * 2))
        return 0;
    const void *w[3];
    const float *bv[3];
    for (int t = 0; t < 3; t++) {
        w[t] = ((const TensorExtra *)mm[t]->src[0]->extra)->packed;
        bv[t] = (const float *)bias[t]->data;
    }
    MI_K_CHECK(mi_qkv_rope_kv_q4_0_batch(ctx->stream, w, n, bv, k, m, x,
                                         norm.w ? (const float *)norm.w->data : nullptr, norm.eps, ctx->scratch,
                                         ctx->scratch_size, R.hd, (const int32_t *)R.pos->data, R.freq_base,
                                         R.freq_scale, R.attn_factor, (float *)R.rope[0]->data, R.sr[0]->data,
                                         R.sr[0]->nb[1], R.sr[1]->data, R.sr[1]->nb[1], R.idx->data,
                                         R.idx->type == GGML_TYPE_I64, std::min(R.sr[0]->ne[1], R.sr[1]->ne[1])));
    return R.last + 1 - i;
}

// Runs node i (and, when fused, the nodes it absorbs); returns the number of nodes consumed.
int compute_node(BackendCtx *ctx, ggml_cgraph *g, int i, const Consumers &C) {
    ggml_tensor *node = ggml_graph_node(g, i);
    const int nn = ggml_graph_n_nodes(g);
    void *st = ctx->stream;
    const bool fuse = ctx->fuse;
    switch (node->op) {
        case GGML_OP_MUL_MAT: {
            if (fuse) {
                if (int used = try_fuse_matmul_add(ctx, g, i, C)) return used;
                if (int used = try_fuse_q4_batch(ctx, g, i, C)) return used;
                if (int used = try_fuse_q8_batch(ctx, g, i, C)) return used;
            }
            // consecutive Q8_0 GEMVs reading the same activation (q/k/v, gate/up): one grouped launch
            if (fuse && packed_fmt(node->src[0]) == GGML_TYPE_Q8_0 && node->src[1]->ne[1] == 1 &&
                node->src[1]->ne[0] <= 4096) {
                ggml_tensor *grp[4] = {node};
                int cnt = 1;
                while (cnt < 4 && i + cnt < nn) {
                    ggml_tensor *nx = ggml_graph_node(g, i + cnt);
                    if (nx->op != GGML_OP_MUL_MAT || nx->src[1] != node->src[1] ||
                        !nx->src[0]->extra || packed_fmt(nx->src[0]) != GGML_TYPE_Q8_0 ||
                        inv_s_of(nx->src[0]) != inv_s_of(node->src[0]))
                        break;
                    grp[cnt++] = nx;
                }
                if (cnt > 1) {
                    for (int j = 0; j < cnt; j++)
                        GGML_ASSERT(((const TensorExtra *)grp[j]->src[0]->extra)->ready);
                    run_mul_mat_q8_group(ctx, grp, cnt);
                    return cnt;
                }
            }
            run_mul_mat(ctx, node);
            return 1;
        }
        case GGML_OP_FLASH_ATTN_EXT:
            if (fuse) {
                if (int used = try_fuse_fa_q4_batch(ctx, g, i, C)) return used;
                if (int used = try_fuse_fa_o(ctx, g, i, C)) return used;
            }
            run_fa(ctx, node);
            return 1;
        case GGML_OP_RMS_NORM: {
            if (fuse) {
                if (int used = try_fuse_persist(ctx, g, i, C)) return used;
                if (int used = try_fuse_attn_in(ctx, g, i, C)) return used;
                if (int used = try_fuse_norm_matmuls(ctx, g, i, C)) return used;
                if (int used = try_fuse_norm_q4_batch(ctx, g, i, C)) return used;
                if (int used = try_fuse_norm_head(ctx, g, i, C)) return used;
            }
            float eps;
            memcpy(&eps, node->op_params, sizeof(float));
            const ggml_tensor *x = node->src[0];
            // RMS_NORM followed by MUL with the norm weight (broadcast row): one launch
            if (fuse && i + 1 < nn) {
                ggml_tensor *nx = ggml_graph_node(g, i + 1);
                if (nx->op == GGML_OP_MUL && nx->src[0] == node && is_f32_contig(nx->src[1]) &&
                    ggml_nelements(nx->src[1]) == x->ne[0] && only_consumed_by(C, node, {nx})) {
                    MI_K_CHECK(mi_rms_norm(st, (const float *)x->data, (const float *)nx->src[1]->data,
                                           (float *)nx->data, x->ne[0], ggml_nrows(x), eps));
                    return 2;
                }
            }
            MI_K_CHECK(mi_rms_norm(st, (const float *)x->data, nullptr, (float *)node->data, x->ne[0], ggml_nrows(x),
                                   eps));
            return 1;
        }
        case GGML_OP_ADD:
        case GGML_OP_MUL: {
            const ggml_tensor *a = node->src[0], *b = node->src[1];
            auto fn = node->op == GGML_OP_ADD ? mi_add_bcast : mi_mul_bcast;
            MI_K_CHECK(fn(st, (const float *)a->data, (const float *)b->data, (float *)node->data, ggml_nelements(a),
                          ggml_nelements(b)));
            return 1;
        }
        case GGML_OP_ROPE: {
            if (fuse) {
                if (int used = try_fuse_rope_kv(ctx, g, i, C)) return used;
            }
            const ggml_tensor *x = node->src[0];
            float freq_base, freq_scale, attn_factor;
            memcpy(&freq_base, (const float *)node->op_params + 5, sizeof(float));
            memcpy(&freq_scale, (const float *)node->op_params + 6, sizeof(float));
            memcpy(&attn_factor, (const float *)node->op_params + 8, sizeof(float));
            MI_K_CHECK(mi_rope_neox(st, (const float *)x->data, (float *)node->data, (const int32_t *)node->src[1]->data,
                                    x->ne[0], x->ne[1], x->ne[2], node->op_params[1], freq_base, freq_scale,
                                    attn_factor, x->nb[1], x->nb[2], node->nb[1], node->nb[2]));
            return 1;
        }
        case GGML_OP_SET_ROWS: {
            const ggml_tensor *src = node->src[0], *idx = node->src[1];
            MI_K_CHECK(mi_set_rows_f16(st, (const float *)src->data, idx->data, idx->type == GGML_TYPE_I64,
                                       (uint16_t *)node->data, src->ne[0], src->ne[1], src->nb[1], node->nb[1],
                                       node->ne[1]));
            return 1;
        }
        case GGML_OP_GET_ROWS: {
            if (fuse)
                if (int used = try_fuse_persist_embd(ctx, g, i, C)) return used;
            const ggml_tensor *src = node->src[0], *idx = node->src[1];
            MI_K_CHECK(mi_get_rows(st, src->data, src->type == GGML_TYPE_F16, (const int32_t *)idx->data,
                                   (float *)node->data, src->ne[0], idx->ne[0], src->nb[1], src->ne[1]));
            return 1;
        }
        case GGML_OP_GLU:
            if (fuse) {
                if (int used = try_fuse_glu_matmul(ctx, g, i, C)) return used;
                if (int used = try_fuse_glu_q4_batch(ctx, g, i, C)) return used;
            }
            MI_K_CHECK(mi_swiglu(st, (const float *)node->src[0]->data, (const float *)node->src[1]->data,
                                 (float *)node->data, ggml_nelements(node)));
            return 1;
        case GGML_OP_ARGMAX: {
            const ggml_tensor *x = node->src[0];
            MI_K_CHECK(mi_argmax(st, (const float *)x->data, (int32_t *)node->data, x->ne[0], ggml_nrows(x),
                                 ctx->scratch, ctx->scratch_size));
            return 1;
        }
        default:
            GGML_ABORT("MI355X: op %s is not supported", ggml_op_name(node->op));
    }
    return 1;
}

void run_graph_nodes(BackendCtx *ctx, ggml_cgraph *g) {
    const int nn = ggml_graph_n_nodes(g);
    const Consumers C = consumers_of(g);
    ctx->rope_key.valid = false;  // the position input may have changed since the last run
    for (int i = 0; i < nn;) {
        ggml_tensor *node = ggml_graph_node(g, i);
        if (is_noop(node)) {
            i++;
            continue;
        }
        if (trace_node_sync())
            fprintf(stderr, "MI355X trace: node=%d name=%s op=%s ne=[%lld,%lld,%lld,%lld] begin\n", i, node->name,
                    ggml_op_name(node->op), (long long)node->ne[0], (long long)node->ne[1], (long long)node->ne[2],
                    (long long)node->ne[3]);
        const int used = compute_node(ctx, g, i, C);
        if (trace_node_sync()) {
            MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
            fprintf(stderr, "MI355X trace: node=%d name=%s op=%s complete (%d node%s)\n", i, node->name,
                    ggml_op_name(node->op), used, used == 1 ? "" : "s");
        }
        i += used;
    }
}

// Everything the captured launches depend on, as a word sequence: per computed node its
// op, type and flags, data pointer, shape, strides and op params; per source its data
// pointer, type, shape and strides (weights also their prepacked copy and SmoothQuant
// divisor).  View nodes launch nothing: what they change reaches the launches through
// their consumers' source entries.  emit(word) returns false to stop the walk.
template <class Emit>
bool walk_signature(ggml_cgraph *g, Emit &&emit) {
    const int nn = ggml_graph_n_nodes(g);
    for (int i = 0; i < nn; i++) {
        const ggml_tensor *t = ggml_graph_node(g, i);
        if (is_noop(t)) continue;
        if (!emit((uint64_t)t->op | ((uint64_t)t->type << 16) | ((uint64_t)(uint32_t)t->flags << 32)) ||
            !emit((uint64_t)(uintptr_t)t->data))
            return false;
        for (int d = 0; d < 4; d++)
            if (!emit((uint64_t)t->ne[d]) || !emit((uint64_t)t->nb[d])) return false;
        for (int p = 0; p < GGML_MAX_OP_PARAMS / 8; p++) {
            uint64_t w;
            memcpy(&w, (const char *)t->op_params + 8 * p, 8);
            if (!emit(w)) return false;
        }
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            const ggml_tensor *src = t->src[s];
            if (!src) continue;
            if (!emit(((uint64_t)s << 56) ^ (uint64_t)(uintptr_t)src->data) || !emit((uint64_t)src->type)) return false;
            for (int d = 0; d < 4; d++)
                if (!emit((uint64_t)src->ne[d])) return false;
            for (int d = 1; d < 4; d++)
                if (!emit((uint64_t)src->nb[d])) return false;
            if (src->extra) {
                const TensorExtra *ex = (const TensorExtra *)src->extra;
                if (!emit((uint64_t)(uintptr_t)ex) || !emit((uint64_t)(uintptr_t)ex->inv_s)) return false;
            }
        }
    }
    return true;
}

// g against the stored signature, reading both and writing nothing (the per-token case)
bool signature_matches(ggml_cgraph *g, const std::vector<uint64_t> &sig) {
    size_t pos = 0;
    const bool walked = walk_signature(g, [&](uint64_t w) { return pos < sig.size() && sig[pos++] == w; });
    return walked && pos == sig.size();
}

void graph_signature(ggml_cgraph *g, std::vector<uint64_t> &sig) {
    sig.clear();
    walk_signature(g, [&](uint64_t w) {
        sig.push_back(w);
        return true;
    });
}

// the last persistent launch's phase timestamps: int32 n_layer, n_wg, n_events, float64
// clock ticks per microsecond, then uint64 [n_layer][n_wg][n_events]
void write_persist_trace(BackendCtx *ctx) {
    int nl = 0, nw = 0, ne = 0;
    double tpu = 0.0;
    if (mi_persist_read_trace(ctx->persist, nullptr, 0, &nl, &nw, &ne, &tpu) != MI_OK) return;
    std::vector<uint64_t> buf((size_t)nl * nw * ne);
    if (mi_persist_read_trace(ctx->persist, buf.data(), buf.size(), nullptr, nullptr, nullptr, nullptr) != MI_OK) {
        fprintf(stderr, "MI355X: persist trace: %s\n", mi_last_error());
        return;
    }
    FILE *f = fopen(ctx->persist_trace.c_str(), "wb");
    if (!f) {
        fprintf(stderr, "MI355X: persist trace: cannot write %s\n", ctx->persist_trace.c_str());
        return;
    }
    const int32_t hdr[3] = {nl, nw, ne};
    fwrite(hdr, sizeof(hdr), 1, f);
    fwrite(&tpu, sizeof(tpu), 1, f);
    fwrite(buf.data(), sizeof(uint64_t), buf.size(), f);
    fclose(f);
}

const char *backend_get_name(ggml_backend_t backend) { return ((BackendCtx *)backend->context)->name.c_str(); }

void backend_free(ggml_backend_t backend) {
    BackendCtx *ctx = (BackendCtx *)backend->context;
    set_device(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->gexec) (void)hipGraphExecDestroy(ctx->gexec);
    if (ctx->persist && !ctx->persist_trace.empty()) write_persist_trace(ctx);
    if (ctx->persist) mi_persist_destroy(ctx->persist);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->fa_ws) (void)hipFree(ctx->fa_ws);
    if (ctx->ffn_counters) (void)hipFree(ctx->ffn_counters);
    for (hipEvent_t e : ctx->pt_ev)
        if (e) (void)hipEventDestroy(e);
    if (ctx->rope_tab) (void)hipFree(ctx->rope_tab);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    delete backend;
}

void backend_set_tensor_async(ggml_backend_t backend, ggml_tensor *tensor, const void *data, size_t offset,
                              size_t size) {
    BackendCtx *ctx = (BackendCtx *)backend->context;
    if (tensor->extra) {  // weights need the side copy: go through the buffer path
        ggml_backend_tensor_set(tensor, data, offset, size);
        return;
    }
    MI_HIP_CHECK(hipMemcpyAsync((char *)tensor->data + offset, data, size, hipMemcpyHostToDevice, ctx->stream));
}

void backend_get_tensor_async(ggml_backend_t backend, const ggml_tensor *tensor, void *data, size_t offset,
                              size_t size) {
    BackendCtx *ctx = (BackendCtx *)backend->context;
    MI_HIP_CHECK(hipMemcpyAsync(data, (const char *)tensor->data + offset, size, hipMemcpyDeviceToHost, ctx->stream));
}

void backend_synchronize(ggml_backend_t backend) {
    BackendCtx *ctx = (BackendCtx *)backend->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    // a persistent launch whose dependency wait gave up has produced invalid results
    if (ctx->persist && mi_persist_status(ctx->persist) != MI_OK) {
        fprintf(stderr, "MI355X: %s\n", mi_last_error());
        ctx->persist_error = true;
    }
}

enum ggml_status backend_graph_compute(ggml_backend_t backend, ggml_cgraph *cgraph) {
    BackendCtx *ctx = (BackendCtx *)backend->context;
    set_device(ctx->device);
    if (ctx->persist && mi_persist_status(ctx->persist) != MI_OK) {
        fprintf(stderr, "MI355X: %s\n", mi_last_error());
        ctx->persist_error = true;
    }
    if (ctx->persist_error) {  // an earlier launch's results were invalid
        ctx->persist_error = false;
        return GGML_STATUS_FAILED;
    }
    ensure_buffers(ctx, cgraph);
    if (!ctx->graphs_on) {
        run_graph_nodes(ctx, cgraph);
        return GGML_STATUS_SUCCESS;
    }
    const bool same = signature_matches(cgraph, ctx->signature);
    if (ctx->gexec && same) {
        MI_HIP_CHECK(hipGraphLaunch(ctx->gexec, ctx->stream));
        return GGML_STATUS_SUCCESS;
    }
    // a changed graph runs eagerly once; when the same graph comes back it is captured
    if (!same) {
        graph_signature(cgraph, ctx->signature);
        ctx->same_calls = 0;
        if (ctx->gexec) {
            MI_HIP_CHECK(hipGraphExecDestroy(ctx->gexec));
            ctx->gexec = nullptr;
        }
        run_graph_nodes(ctx, cgraph);
        return GGML_STATUS_SUCCESS;
    }
    hipGraph_t graph = nullptr;
    MI_HIP_CHECK(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    run_graph_nodes(ctx, cgraph);
    MI_HIP_CHECK(hipStreamEndCapture(ctx->stream, &graph));
    MI_HIP_CHECK(hipGraphInstantiate(&ctx->gexec, graph, nullptr, nullptr, 0));
    MI_HIP_CHECK(hipGraphDestroy(graph));
    MI_HIP_CHECK(hipGraphLaunch(ctx->gexec, ctx->stream));
    return GGML_STATUS_SUCCESS;
}

const ggml_backend_i kBackendIface = {
    /* get_name           */ backend_get_name,
    /* free               */ backend_free,
    /* set_tensor_async   */ backend_set_tensor_async,
    /* get_tensor_async   */ backend_get_tensor_async,
    /* cpy_tensor_async   */ nullptr,
    /* synchronize        */ backend_synchronize,
    /* graph_plan_create  */ nullptr,
    /* graph_plan_free    */ nullptr,
    /* graph_plan_update  */ nullptr,
    /* graph_plan_compute */ nullptr,
    /* graph_compute      */ backend_graph_compute,
    /* event_record       */ nullptr,
    /* event_wait         */ nullptr,
    /* graph_optimize     */ nullptr,
};

ggml_guid_t backend_guid() {
    static ggml_guid guid = {{0x6d, 0x69, 0x33, 0x35, 0x35, 0x78, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x2d,
                              0x76, 0x31}};
    return &guid;
}

// ---- device iface

const char *dev_get_name(ggml_backend_dev_t dev) { return ((DeviceCtx *)dev->context)->name.c_str(); }
const char *dev_get_description(ggml_backend_dev_t dev) { return ((DeviceCtx *)dev->context)->description.c_str(); }

void dev_get_memory(ggml_backend_dev_t dev, size_t *free, size_t *total) {
    set_device(((DeviceCtx *)dev->context)->device);
    MI_HIP_CHECK(hipMemGetInfo(free, total));
}

enum ggml_backend_dev_type dev_get_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_get_props(ggml_backend_dev_t dev, ggml_backend_dev_props *props) {
    props->name = dev_get_name(dev);
    props->description = dev_get_description(dev);
    props->type = GGML_BACKEND_DEVICE_TYPE_GPU;
    props->device_id = nullptr;
    dev_get_memory(dev, &props->memory_free, &props->memory_total);
    props->caps = {/* async */ true, /* host_buffer */ false, /* buffer_from_host_ptr */ false, /* events */ false};
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t dev, const char *) {
    return ggml_backend_mi355x_init(((DeviceCtx *)dev->context)->device);
}

ggml_backend_buffer_type_t dev_get_buffer_type(ggml_backend_dev_t dev) { return &((DeviceCtx *)dev->context)->buft; }

bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor *op) { return supports_op_impl(op); }

bool dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft) {
    return buft->iface.get_name == buft_get_name && buft->context == dev->context;
}

bool dev_offload_op(ggml_backend_dev_t, const ggml_tensor *) { return false; }

const ggml_backend_device_i kDeviceIface = {
    /* get_name             */ dev_get_name,
    /* get_description      */ dev_get_description,
    /* get_memory           */ dev_get_memory,
    /* get_type             */ dev_get_type,
    /* get_props            */ dev_get_props,
    /* init_backend         */ dev_init_backend,
    /* get_buffer_type      */ dev_get_buffer_type,
    /* get_host_buffer_type */ nullptr,
    /* buffer_from_host_ptr */ nullptr,
    /* supports_op          */ dev_supports_op,
    /* supports_buft        */ dev_supports_buft,
    /* offload_op           */ dev_offload_op,
    /* event_new            */ nullptr,
    /* event_free           */ nullptr,
    /* event_synchronize    */ nullptr,
};

// ---- registry

struct RegCtx {
    std::vector<std::unique_ptr<DeviceCtx>> dev_ctx;
    std::vector<std::unique_ptr<ggml_backend_device>> devs;
};

const char *reg_get_name(ggml_backend_reg_t) { return GGML_MI355X_NAME; }
size_t reg_get_device_count(ggml_backend_reg_t reg) { return ((RegCtx *)reg->context)->devs.size(); }
ggml_backend_dev_t reg_get_device(ggml_backend_reg_t reg, size_t index) {
    RegCtx *ctx = (RegCtx *)reg->context;
    GGML_ASSERT(index < ctx->devs.size());
    return ctx->devs[index].get();
}
void *reg_get_proc_address(ggml_backend_reg_t, const char *name) {
    if (strcmp(name, "ggml_backend_mi355x_set_smooth_factors") == 0) return (void *)ggml_backend_mi355x_set_smooth_factors;
    return nullptr;
}

const ggml_backend_reg_i kRegIface = {reg_get_name, reg_get_device_count, reg_get_device, reg_get_proc_address};

RegCtx *registry_ctx() {
    static RegCtx *ctx = [] {
        RegCtx *c = new RegCtx();
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        for (int i = 0; i < n && i < GGML_MI355X_MAX_DEVICES; i++) {
            auto d = std::make_unique<DeviceCtx>();
            d->device = i;
            d->name = std::string(GGML_MI355X_NAME) + std::to_string(i);
            hipDeviceProp_t p;
            if (hipGetDeviceProperties(&p, i) == hipSuccess)
                d->description = std::string(p.name) + " (" + p.gcnArchName + ")";
            else
                d->description = "HIP device";
            d->buft_name = d->name;
            d->buft.iface = kBuftIface;
            d->buft.context = d.get();
            auto dev = std::make_unique<ggml_backend_device>();
            dev->iface = kDeviceIface;
            dev->reg = nullptr;
            dev->context = d.get();
            d->buft.device = dev.get();
            c->dev_ctx.push_back(std::move(d));
            c->devs.push_back(std::move(dev));
        }
        return c;
    }();
    return ctx;
}

}  // namespace

extern "C" {

ggml_backend_reg_t ggml_backend_mi355x_reg(void) {
    static ggml_backend_reg reg = [] {
        ggml_backend_reg r;
        r.api_version = GGML_BACKEND_API_VERSION;
        r.iface = kRegIface;
        r.context = registry_ctx();
        return r;
    }();
    static std::once_flag once;
    std::call_once(once, [] {
        for (auto &d : registry_ctx()->devs) d->reg = &reg;
    });
    return &reg;
}

int ggml_backend_mi355x_get_device_count(void) { return (int)registry_ctx()->devs.size(); }

void ggml_backend_mi355x_get_device_description(int device, char *description, size_t description_size) {
    RegCtx *c = registry_ctx();
    if (device < 0 || device >= (int)c->dev_ctx.size()) {
        snprintf(description, description_size, "invalid device");
        return;
    }
    snprintf(description, description_size, "%s", c->dev_ctx[device]->description.c_str());
}

void ggml_backend_mi355x_get_device_memory(int device, size_t *free, size_t *total) {
    set_device(device);
    MI_HIP_CHECK(hipMemGetInfo(free, total));
}

ggml_backend_buffer_type_t ggml_backend_mi355x_buffer_type(int device) {
    ggml_backend_mi355x_reg();
    RegCtx *c = registry_ctx();
    if (device < 0 || device >= (int)c->dev_ctx.size()) return nullptr;
    return &c->dev_ctx[device]->buft;
}

ggml_backend_t ggml_backend_mi355x_init(int device) {
    ggml_backend_reg_t reg = ggml_backend_mi355x_reg();
    RegCtx *c = registry_ctx();
    if (device < 0 || device >= (int)c->devs.size()) {
        fprintf(stderr, "MI355X: invalid device %d\n", device);
        return nullptr;
    }
    (void)reg;
    set_device(device);
    BackendCtx *ctx = new BackendCtx();
    ctx->device = device;
    ctx->fuse = fusion_env();
    ctx->persist_on = env_flag("GGML_MI355X_PERSIST", false);
    if (const char *tp = getenv("GGML_MI355X_PERSIST_TRACE")) ctx->persist_trace = tp;
    ctx->persist_timing = env_flag("GGML_MI355X_PERSIST_TIMING", false);
    ctx->graphs_on = graphs_env();
    if (ctx->persist_timing)
        for (hipEvent_t &e : ctx->pt_ev) MI_HIP_CHECK(hipEventCreate(&e));
    ctx->name = std::string(GGML_MI355X_NAME) + std::to_string(device);
    MI_HIP_CHECK(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    return new ggml_backend{backend_guid(), kBackendIface, c->devs[device].get(), ctx};
}

bool ggml_backend_is_mi355x(ggml_backend_t backend) {
    return backend != nullptr && backend->guid == backend_guid();
}

int ggml_backend_mi355x_status(ggml_backend_t backend) {
    if (!ggml_backend_is_mi355x(backend)) return -1;
    BackendCtx *ctx = (BackendCtx *)backend->context;
    set_device(ctx->device);
    MI_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    collect_persist_timing(ctx);
    if (ctx->persist && mi_persist_status(ctx->persist) != MI_OK) ctx->persist_error = true;
    if (!ctx->persist_error) return 0;
    ctx->persist_error = false;
    return -1;
}

int ggml_backend_mi355x_persist_timing(ggml_backend_t backend, int64_t *launches, double *total_ms) {
    if (!ggml_backend_is_mi355x(backend) || !launches || !total_ms) return -1;
    const BackendCtx *ctx = (const BackendCtx *)backend->context;
    *launches = ctx->pt_launches;
    *total_ms = ctx->pt_ms;
    return ctx->persist_timing ? 0 : -1;
}

bool ggml_backend_mi355x_set_smooth_factors(struct ggml_tensor *weight, const float *s, int64_t n) {
    // only weights of this backend's buffers carry a TensorExtra (CPU extra buffer types
    // hang their own data on tensor->extra)
    if (!weight || !s || n != weight->ne[0] || !weight->buffer ||
        weight->buffer->buft->iface.get_alloc_size != buft_get_alloc_size)
        return false;
    for (int64_t i = 0; i < n; i++)
        if (!(s[i] > 0.0f) || !isfinite(s[i])) return false;
    // an unquantized F16 weight (a layer kept F16, or A8W8 off): (x/s) . W*diag(s) is W.x,
    // so there is nothing to fold in or divide by
    if (!weight->extra) return weight->type == GGML_TYPE_F16;
    TensorExtra *ex = (TensorExtra *)weight->extra;
    if (ex->fmt != GGML_TYPE_Q8_0) return false;  // W4A16 quantizes no activation
    BufferCtx *bctx = (BufferCtx *)weight->buffer->context;
    std::vector<float> inv((size_t)n);
    for (int64_t i = 0; i < n; i++) inv[i] = 1.0f / s[i];
    const float *dev_inv = upload_factors(bctx, inv.data(), n);
    const float *dev_s = weight->type == GGML_TYPE_F16 ? upload_factors(bctx, s, n) : nullptr;
    std::lock_guard<std::mutex> lk(ex->mtx);
    ex->inv_s = dev_inv;
    if (weight->type == GGML_TYPE_F16) {
        ex->s = dev_s;
        if (ex->ready) build_side_copy_locked(bctx, weight);  // re-quantize W*diag(s)
    }
    return true;
}

// The backend dispatches on enum ggml_op / ggml_type values compiled in from the ggml
// headers it was built against.  Loaded dynamically it runs inside the host process's
// libggml-base, whose op and type tables must give those values the same names;
// otherwise the two were built from different ggml revisions and every id could mean
// another op (an upstream DIV read as MUL_MAT).
int ggml_backend_mi355x_abi_check(char *msg, size_t msg_size) {
    struct Id {
        bool is_op;
        int value;
        const char *name;
    };
    static const Id ids[] = {
        {true, GGML_OP_NONE, "NONE"},         {true, GGML_OP_ADD, "ADD"},
        {true, GGML_OP_MUL, "MUL"},           {true, GGML_OP_RMS_NORM, "RMS_NORM"},
        {true, GGML_OP_MUL_MAT, "MUL_MAT"},   {true, GGML_OP_RESHAPE, "RESHAPE"},
        {true, GGML_OP_VIEW, "VIEW"},         {true, GGML_OP_PERMUTE, "PERMUTE"},
        {true, GGML_OP_TRANSPOSE, "TRANSPOSE"}, {true, GGML_OP_GET_ROWS, "GET_ROWS"},
        {true, GGML_OP_SET_ROWS, "SET_ROWS"}, {true, GGML_OP_ROPE, "ROPE"},
        {true, GGML_OP_FLASH_ATTN_EXT, "FLASH_ATTN_EXT"}, {true, GGML_OP_GLU, "GLU"},
        {true, GGML_OP_ARGMAX, "ARGMAX"},
        {false, GGML_TYPE_F32, "f32"},        {false, GGML_TYPE_F16, "f16"},
        {false, GGML_TYPE_Q4_0, "q4_0"},      {false, GGML_TYPE_Q8_0, "q8_0"},
        {false, GGML_TYPE_I32, "i32"},        {false, GGML_TYPE_I64, "i64"},
    };
    for (const Id &id : ids) {
        const char *got = id.is_op ? ggml_op_name((enum ggml_op)id.value) : ggml_type_name((enum ggml_type)id.value);
        if (!got || strcmp(got, id.name) != 0) {
            if (msg && msg_size)
                snprintf(msg, msg_size, "ggml %s id %d is %s in the loaded ggml, %s in this backend's build",
                         id.is_op ? "op" : "type", id.value, got ? got : "(null)", id.name);
            return 0;
        }
    }
    if (msg && msg_size) snprintf(msg, msg_size, "ok: %zu op and type ids agree", sizeof(ids) / sizeof(ids[0]));
    return 1;
}

#ifdef GGML_BACKEND_DL
// the entry points ggml's dynamic backend loader resolves (GGML_BACKEND_DL_IMPL /
// GGML_BACKEND_DL_SCORE_IMPL of ggml-backend-impl.h)
ggml_backend_reg_t ggml_backend_init(void) {
    char msg[256];
    if (!ggml_backend_mi355x_abi_check(msg, sizeof(msg))) {
        fprintf(stderr, "MI355X: not registering: %s\n", msg);
        return nullptr;
    }
    return ggml_backend_mi355x_reg();
}

// 0 (not usable) without a gfx950 device or with mismatched ggml ids
int ggml_backend_score(void) {
    if (!ggml_backend_mi355x_abi_check(nullptr, 0)) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && strncmp(p.gcnArchName, "gfx950", 6) == 0) return 100;
    }
    return 0;
}
#endif

}  // extern "C"

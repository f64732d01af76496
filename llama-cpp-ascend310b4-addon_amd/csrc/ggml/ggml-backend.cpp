// ggml-backend.cpp -- the generic half of the restated ggml backend API: thin
// dispatch through the plugin vtables (ggml-backend-impl.h) plus the two
// allocators a model loader and a graph runner need.
#include "ggml-backend-impl.h"

#include <stdlib.h>
#include <string.h>

#include <vector>

extern "C" {

// ---------------------------------------------------------------- buffer types

const char *ggml_backend_buft_name(ggml_backend_buffer_type_t buft) { return buft->iface.get_name(buft); }

ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    return buft->iface.alloc_buffer(buft, size);
}

size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft) { return buft->iface.get_alignment(buft); }

size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor *tensor) {
    if (buft->iface.get_alloc_size) return buft->iface.get_alloc_size(buft, tensor);
    return ggml_nbytes(tensor);
}

bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft) {
    return buft->iface.is_host ? buft->iface.is_host(buft) : false;
}

// ---------------------------------------------------------------- buffers

ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void *context, size_t size) {
    ggml_backend_buffer_t b = new ggml_backend_buffer{iface, buft, context, size, GGML_BACKEND_BUFFER_USAGE_ANY};
    return b;
}

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) return;
    if (buffer->iface.free_buffer) buffer->iface.free_buffer(buffer);
    delete buffer;
}

void *ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer) { return buffer->iface.get_base(buffer); }
size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer->size; }

enum ggml_status ggml_backend_buffer_init_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor) {
    if (buffer->iface.init_tensor) return buffer->iface.init_tensor(buffer, tensor);
    return GGML_STATUS_SUCCESS;
}

void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) { buffer->iface.clear(buffer, value); }

void ggml_backend_buffer_set_usage(ggml_backend_buffer_t buffer, enum ggml_backend_buffer_usage usage) {
    buffer->usage = usage;
}

enum ggml_backend_buffer_usage ggml_backend_buffer_get_usage(ggml_backend_buffer_t buffer) { return buffer->usage; }
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) { return buffer->buft; }

size_t ggml_backend_buffer_get_alloc_size(ggml_backend_buffer_t buffer, const struct ggml_tensor *tensor) {
    return ggml_backend_buft_get_alloc_size(buffer->buft, tensor);
}

// ---------------------------------------------------------------- tensor data

void ggml_backend_tensor_set(struct ggml_tensor *tensor, const void *data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor->view_src ? tensor->view_src->buffer : tensor->buffer;
    GGML_ASSERT(buf != nullptr && "tensor buffer not set");
    GGML_ASSERT(tensor->data != nullptr && "tensor not allocated");
    GGML_ASSERT(offset + size <= ggml_nbytes(tensor) && "tensor write out of bounds");
    if (size == 0) return;
    buf->iface.set_tensor(buf, tensor, data, offset, size);
}

// ggml-backend.h: the backend's asynchronous copy when it has one (ordered with its
// graph_compute calls; data must stay valid until ggml_backend_synchronize), else the
// buffer's synchronous copy
void ggml_backend_tensor_set_async(ggml_backend_t backend, struct ggml_tensor *tensor, const void *data, size_t offset,
                                   size_t size) {
    GGML_ASSERT(tensor->data != nullptr && "tensor not allocated");
    GGML_ASSERT(offset + size <= ggml_nbytes(tensor) && "tensor write out of bounds");
    if (size == 0) return;
    if (backend->iface.set_tensor_async == nullptr) ggml_backend_tensor_set(tensor, data, offset, size);
    else backend->iface.set_tensor_async(backend, tensor, data, offset, size);
}

void ggml_backend_tensor_get_async(ggml_backend_t backend, const struct ggml_tensor *tensor, void *data,
                                   size_t offset, size_t size) {
    GGML_ASSERT(tensor->data != nullptr && "tensor not allocated");
    GGML_ASSERT(offset + size <= ggml_nbytes(tensor) && "tensor read out of bounds");
    if (size == 0) return;
    if (backend->iface.get_tensor_async == nullptr) ggml_backend_tensor_get(tensor, data, offset, size);
    else backend->iface.get_tensor_async(backend, tensor, data, offset, size);
}

void ggml_backend_tensor_get(const struct ggml_tensor *tensor, void *data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor->view_src ? tensor->view_src->buffer : tensor->buffer;
    GGML_ASSERT(buf != nullptr && "tensor buffer not set");
    GGML_ASSERT(tensor->data != nullptr && "tensor not allocated");
    GGML_ASSERT(offset + size <= ggml_nbytes(tensor) && "tensor read out of bounds");
    if (size == 0) return;
    buf->iface.get_tensor(buf, tensor, data, offset, size);
}

void ggml_backend_tensor_memset(struct ggml_tensor *tensor, uint8_t value, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor->view_src ? tensor->view_src->buffer : tensor->buffer;
    GGML_ASSERT(buf != nullptr && buf->iface.memset_tensor != nullptr);
    GGML_ASSERT(offset + size <= ggml_nbytes(tensor));
    if (size == 0) return;
    buf->iface.memset_tensor(buf, tensor, value, offset, size);
}

// ---------------------------------------------------------------- backends

const char *ggml_backend_name(ggml_backend_t backend) { return backend->iface.get_name(backend); }

void ggml_backend_free(ggml_backend_t backend) {
    if (backend) backend->iface.free(backend);
}

ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend) {
    return ggml_backend_dev_buffer_type(backend->device);
}

void ggml_backend_synchronize(ggml_backend_t backend) {
    if (backend->iface.synchronize) backend->iface.synchronize(backend);
}

enum ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, struct ggml_cgraph *cgraph) {
    return backend->iface.graph_compute(backend, cgraph);
}

enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph *cgraph) {
    const enum ggml_status st = ggml_backend_graph_compute_async(backend, cgraph);
    ggml_backend_synchronize(backend);
    return st;
}

bool ggml_backend_supports_op(ggml_backend_t backend, const struct ggml_tensor *op) {
    return ggml_backend_dev_supports_op(backend->device, op);
}

ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend) { return backend->device; }

// ---------------------------------------------------------------- devices / registries

const char *ggml_backend_dev_name(ggml_backend_dev_t d) { return d->iface.get_name(d); }
const char *ggml_backend_dev_description(ggml_backend_dev_t d) { return d->iface.get_description(d); }
void ggml_backend_dev_get_memory(ggml_backend_dev_t d, size_t *free, size_t *total) { d->iface.get_memory(d, free, total); }
enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t d) { return d->iface.get_type(d); }
void ggml_backend_dev_get_props(ggml_backend_dev_t d, struct ggml_backend_dev_props *p) { d->iface.get_props(d, p); }
ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t d, const char *params) { return d->iface.init_backend(d, params); }
ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t d) { return d->iface.get_buffer_type(d); }
bool ggml_backend_dev_supports_op(ggml_backend_dev_t d, const struct ggml_tensor *op) { return d->iface.supports_op(d, op); }
bool ggml_backend_dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t b) { return d->iface.supports_buft(d, b); }

const char *ggml_backend_reg_name(ggml_backend_reg_t reg) { return reg->iface.get_name(reg); }
size_t ggml_backend_reg_dev_count(ggml_backend_reg_t reg) { return reg->iface.get_device_count(reg); }
ggml_backend_dev_t ggml_backend_reg_dev_get(ggml_backend_reg_t reg, size_t index) {
    return reg->iface.get_device(reg, index);
}
void *ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char *name) {
    return reg->iface.get_proc_address ? reg->iface.get_proc_address(reg, name) : nullptr;
}

// ---------------------------------------------------------------- host-memory buffer type
// (upstream's ggml_backend_cpu_buffer_type lives in ggml-base too: plain aligned host
// memory, set/get are copies; its device is NULL)

namespace {
constexpr size_t kHostAlign = 64;

void host_free_buffer(ggml_backend_buffer_t b) { free(b->context); }
void *host_get_base(ggml_backend_buffer_t b) { return b->context; }
void host_memset_tensor(ggml_backend_buffer_t, struct ggml_tensor *t, uint8_t v, size_t off, size_t size) {
    memset((char *)t->data + off, v, size);
}
void host_set_tensor(ggml_backend_buffer_t, struct ggml_tensor *t, const void *data, size_t off, size_t size) {
    memcpy((char *)t->data + off, data, size);
}
void host_get_tensor(ggml_backend_buffer_t, const struct ggml_tensor *t, void *data, size_t off, size_t size) {
    memcpy(data, (const char *)t->data + off, size);
}
void host_clear(ggml_backend_buffer_t b, uint8_t v) { memset(b->context, v, b->size); }

const ggml_backend_buffer_i kHostBufferIface = {host_free_buffer, host_get_base, nullptr, host_memset_tensor,
                                                host_set_tensor, host_get_tensor, nullptr, host_clear, nullptr};

const char *host_buft_name(ggml_backend_buffer_type_t) { return "CPU"; }
ggml_backend_buffer_t host_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    void *p = aligned_alloc(kHostAlign, GGML_PAD(size ? size : 1, kHostAlign));
    return p ? ggml_backend_buffer_init(buft, kHostBufferIface, p, size) : nullptr;
}
size_t host_alignment(ggml_backend_buffer_type_t) { return kHostAlign; }
bool host_is_host(ggml_backend_buffer_type_t) { return true; }
}  // namespace

ggml_backend_buffer_type_t ggml_backend_cpu_buffer_type(void) {
    static ggml_backend_buffer_type buft = {
        {host_buft_name, host_alloc_buffer, host_alignment, nullptr, nullptr, host_is_host}, nullptr, nullptr};
    return &buft;
}

// ---------------------------------------------------------------- allocation

enum ggml_status ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, struct ggml_tensor *tensor, void *addr) {
    GGML_ASSERT(tensor->buffer == nullptr && tensor->data == nullptr && tensor->view_src == nullptr);
    tensor->buffer = buffer;
    tensor->data = addr;
    return ggml_backend_buffer_init_tensor(buffer, tensor);
}

enum ggml_status ggml_backend_view_init(struct ggml_tensor *tensor) {
    GGML_ASSERT(tensor->view_src != nullptr && tensor->view_src->data != nullptr);
    tensor->buffer = tensor->view_src->buffer;
    tensor->data = (char *)tensor->view_src->data + tensor->view_offs;
    return ggml_backend_buffer_init_tensor(tensor->buffer, tensor);
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context *ctx,
                                                               ggml_backend_buffer_type_t buft) {
    const size_t align = ggml_backend_buft_get_alignment(buft);
    size_t total = 0;
    for (ggml_tensor *t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data || t->view_src) continue;
        total = GGML_PAD(total, align) + ggml_backend_buft_get_alloc_size(buft, t);
    }
    if (total == 0) return nullptr;
    ggml_backend_buffer_t buf = ggml_backend_buft_alloc_buffer(buft, total);
    if (!buf) return nullptr;
    char *base = (char *)ggml_backend_buffer_get_base(buf);
    size_t off = 0;
    for (ggml_tensor *t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data || t->view_src) continue;
        off = GGML_PAD(off, align);
        if (ggml_backend_tensor_alloc(buf, t, base + off) != GGML_STATUS_SUCCESS) {
            ggml_backend_buffer_free(buf);
            return nullptr;
        }
        off += ggml_backend_buft_get_alloc_size(buft, t);
    }
    for (ggml_tensor *t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t))
        if (t->view_src && !t->data && t->view_src->data) ggml_backend_view_init(t);
    return buf;
}

struct ggml_gallocr {
    ggml_backend_buffer_type_t buft;
    ggml_backend_buffer_t buffer = nullptr;
};

ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft) {
    ggml_gallocr *g = new ggml_gallocr();
    g->buft = buft;
    return g;
}

void ggml_gallocr_free(ggml_gallocr_t galloc) {
    if (!galloc) return;
    ggml_backend_buffer_free(galloc->buffer);
    delete galloc;
}

bool ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph *graph) {
    const size_t align = ggml_backend_buft_get_alignment(galloc->buft);
    std::vector<ggml_tensor *> todo;
    auto want = [&](ggml_tensor *t) {
        if (t && !t->data && !t->view_src) todo.push_back(t);
    };
    for (int i = 0; i < ggml_graph_n_leafs(graph); i++) want(ggml_graph_leaf(graph, i));
    for (int i = 0; i < ggml_graph_n_nodes(graph); i++) want(ggml_graph_node(graph, i));
    size_t total = 0;
    for (ggml_tensor *t : todo) total = GGML_PAD(total, align) + ggml_backend_buft_get_alloc_size(galloc->buft, t);
    if (total > 0) {
        ggml_backend_buffer_free(galloc->buffer);
        galloc->buffer = ggml_backend_buft_alloc_buffer(galloc->buft, total);
        if (!galloc->buffer) return false;
        ggml_backend_buffer_set_usage(galloc->buffer, GGML_BACKEND_BUFFER_USAGE_COMPUTE);
        char *base = (char *)ggml_backend_buffer_get_base(galloc->buffer);
        size_t off = 0;
        for (ggml_tensor *t : todo) {
            off = GGML_PAD(off, align);
            if (ggml_backend_tensor_alloc(galloc->buffer, t, base + off) != GGML_STATUS_SUCCESS) return false;
            off += ggml_backend_buft_get_alloc_size(galloc->buft, t);
        }
    }
    // views (in graph order, so chains resolve front to back)
    for (int i = 0; i < ggml_graph_n_leafs(graph); i++) {
        ggml_tensor *t = ggml_graph_leaf(graph, i);
        if (t->view_src && !t->data) ggml_backend_view_init(t);
    }
    for (int i = 0; i < ggml_graph_n_nodes(graph); i++) {
        ggml_tensor *t = ggml_graph_node(graph, i);
        if (t->view_src && !t->data) ggml_backend_view_init(t);
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            ggml_tensor *src = t->src[s];
            if (src && src->view_src && !src->data && src->view_src->data) ggml_backend_view_init(src);
        }
    }
    return true;
}

}  // extern "C"

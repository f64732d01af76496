// ggml.cpp -- implementation of the restated ggml tensor/graph subset (see ggml.h).
// Tensor headers live in a per-context list; tensor data (when the context
// allocates) in per-tensor aligned blocks; views and graph construction follow
// upstream ggml's rules (view_src chains collapse, DFS graph order with
// sources visited first, NONE-op tensors become leafs).
#include "ggml.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <deque>
#include <memory>
#include <string>
#include <unordered_set>
#include <vector>

struct ggml_context {
    bool no_alloc = true;
    std::deque<ggml_tensor> tensors;
    std::vector<void *> blocks;
    std::deque<ggml_cgraph> graphs;
};

struct ggml_cgraph {
    int size = 0;
    std::vector<ggml_tensor *> nodes;
    std::vector<ggml_tensor *> leafs;
    std::unordered_set<const ggml_tensor *> visited;
};

extern "C" {

void ggml_abort(const char *file, int line, const char *fmt, ...) {
    fprintf(stderr, "%s:%d: ", file, line);
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stderr, fmt, ap);
    va_end(ap);
    fprintf(stderr, "\n");
    abort();
}

// ---------------------------------------------------------------- fp16 (RNE)

float ggml_fp16_to_fp32(ggml_fp16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            e = 113;
            while (!(m & 0x400u)) { m <<= 1; e--; }
            x = sign | (e << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

ggml_fp16_t ggml_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (ggml_fp16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (ggml_fp16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax <= 0x33000000u) return (ggml_fp16_t)sign;
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126u - e;
        uint32_t h = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (ggml_fp16_t)(sign | h);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (ggml_fp16_t)(sign | h);
}

// ---------------------------------------------------------------- types

int64_t ggml_blck_size(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_Q4_0: case GGML_TYPE_Q4_1: case GGML_TYPE_Q5_0: case GGML_TYPE_Q5_1:
        case GGML_TYPE_Q8_0: case GGML_TYPE_Q8_1: return 32;
        default: return 1;
    }
}

size_t ggml_type_size(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_F32: return 4;
        case GGML_TYPE_F16: return 2;
        case GGML_TYPE_BF16: return 2;
        case GGML_TYPE_Q4_0: return 18;
        case GGML_TYPE_Q4_1: return 20;
        case GGML_TYPE_Q5_0: return 22;
        case GGML_TYPE_Q5_1: return 24;
        case GGML_TYPE_Q8_0: return 34;
        case GGML_TYPE_Q8_1: return 36;
        case GGML_TYPE_I8: return 1;
        case GGML_TYPE_I16: return 2;
        case GGML_TYPE_I32: return 4;
        case GGML_TYPE_I64: return 8;
        case GGML_TYPE_F64: return 8;
        default: GGML_ABORT("ggml_type_size: unsupported type %d", (int)type);
    }
}

size_t ggml_row_size(enum ggml_type type, int64_t ne) {
    GGML_ASSERT(ne % ggml_blck_size(type) == 0);
    return ggml_type_size(type) * (size_t)(ne / ggml_blck_size(type));
}

bool ggml_is_quantized(enum ggml_type type) { return ggml_blck_size(type) > 1; }

const char *ggml_type_name(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_F32: return "f32";
        case GGML_TYPE_F16: return "f16";
        case GGML_TYPE_BF16: return "bf16";
        case GGML_TYPE_Q4_0: return "q4_0";
        case GGML_TYPE_Q4_1: return "q4_1";
        case GGML_TYPE_Q5_0: return "q5_0";
        case GGML_TYPE_Q5_1: return "q5_1";
        case GGML_TYPE_Q8_0: return "q8_0";
        case GGML_TYPE_Q8_1: return "q8_1";
        case GGML_TYPE_I8: return "i8";
        case GGML_TYPE_I16: return "i16";
        case GGML_TYPE_I32: return "i32";
        case GGML_TYPE_I64: return "i64";
        case GGML_TYPE_F64: return "f64";
        default: return "?";
    }
}

const char *ggml_op_name(enum ggml_op op) {
    static const char *names[GGML_OP_COUNT] = {
        "NONE", "DUP", "ADD", "SUB", "MUL", "DIV", "ARGMAX", "RMS_NORM", "MUL_MAT", "SCALE", "CPY", "CONT",
        "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS", "SET_ROWS", "SOFT_MAX", "ROPE", "FLASH_ATTN_EXT",
        "UNARY", "GLU"};
    return (op >= 0 && op < GGML_OP_COUNT) ? names[op] : "?";
}

int64_t ggml_nelements(const struct ggml_tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t ggml_nrows(const struct ggml_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

size_t ggml_nbytes(const struct ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] <= 0) return 0;
    const int64_t blck = ggml_blck_size(t->type);
    size_t nbytes;
    if (blck == 1) {
        nbytes = ggml_type_size(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; i++) nbytes += (size_t)(t->ne[i] - 1) * t->nb[i];
    } else {
        nbytes = (size_t)(t->ne[0] * t->nb[0] / blck);
        for (int i = 1; i < GGML_MAX_DIMS; i++) nbytes += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return nbytes;
}

bool ggml_is_contiguous(const struct ggml_tensor *t) {
    size_t next_nb = ggml_type_size(t->type);
    if (t->ne[0] != ggml_blck_size(t->type) && t->nb[0] != next_nb) return false;
    next_nb *= (size_t)(t->ne[0] / ggml_blck_size(t->type));
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1) {
            if (t->nb[i] != next_nb) return false;
            next_nb *= (size_t)t->ne[i];
        }
    }
    return true;
}

bool ggml_is_empty(const struct ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] == 0) return true;
    return false;
}

bool ggml_are_same_shape(const struct ggml_tensor *a, const struct ggml_tensor *b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}

enum ggml_unary_op ggml_get_unary_op(const struct ggml_tensor *t) { return (enum ggml_unary_op)t->op_params[0]; }
enum ggml_glu_op ggml_get_glu_op(const struct ggml_tensor *t) { return (enum ggml_glu_op)t->op_params[0]; }

// ---------------------------------------------------------------- context

struct ggml_context *ggml_init(struct ggml_init_params params) {
    ggml_context *ctx = new ggml_context();
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

void ggml_free(struct ggml_context *ctx) {
    if (!ctx) return;
    for (void *b : ctx->blocks) free(b);
    delete ctx;
}

bool ggml_get_no_alloc(struct ggml_context *ctx) { return ctx->no_alloc; }

struct ggml_tensor *ggml_get_first_tensor(const struct ggml_context *ctx) {
    return ctx->tensors.empty() ? nullptr : const_cast<ggml_tensor *>(&ctx->tensors.front());
}

struct ggml_tensor *ggml_get_next_tensor(const struct ggml_context *ctx, struct ggml_tensor *tensor) {
    for (size_t i = 0; i + 1 < ctx->tensors.size(); i++)
        if (&ctx->tensors[i] == tensor) return const_cast<ggml_tensor *>(&ctx->tensors[i + 1]);
    return nullptr;
}

struct ggml_tensor *ggml_get_tensor(struct ggml_context *ctx, const char *name) {
    for (auto &t : ctx->tensors)
        if (strcmp(t.name, name) == 0) return &t;
    return nullptr;
}

static ggml_tensor *new_tensor_impl(ggml_context *ctx, ggml_type type, int n_dims, const int64_t *ne,
                                    ggml_tensor *view_src, size_t view_offs) {
    GGML_ASSERT(n_dims >= 1 && n_dims <= GGML_MAX_DIMS);
    if (view_src && view_src->view_src) {
        view_offs += view_src->view_offs;
        view_src = view_src->view_src;
    }
    ctx->tensors.emplace_back();
    ggml_tensor *t = &ctx->tensors.back();
    memset(t, 0, sizeof(*t));
    t->type = type;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->ne[i] = i < n_dims ? ne[i] : 1;
    t->nb[0] = ggml_type_size(type);
    t->nb[1] = t->nb[0] * (size_t)(t->ne[0] / ggml_blck_size(type));
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t)t->ne[i - 1];
    t->op = GGML_OP_NONE;
    t->view_src = view_src;
    t->view_offs = view_offs;
    if (view_src) {
        t->buffer = view_src->buffer;
        if (view_src->data) t->data = (char *)view_src->data + view_offs;
    } else if (!ctx->no_alloc) {
        const size_t sz = GGML_PAD(ggml_nbytes(t), GGML_MEM_ALIGN);
        void *p = nullptr;
        if (posix_memalign(&p, 64, sz ? sz : 64) != 0) GGML_ABORT("ggml: out of host memory");
        ctx->blocks.push_back(p);
        t->data = p;
    }
    return t;
}

struct ggml_tensor *ggml_new_tensor(struct ggml_context *ctx, enum ggml_type type, int n_dims, const int64_t *ne) {
    return new_tensor_impl(ctx, type, n_dims, ne, nullptr, 0);
}
struct ggml_tensor *ggml_new_tensor_1d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0) {
    return ggml_new_tensor(ctx, type, 1, &ne0);
}
struct ggml_tensor *ggml_new_tensor_2d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return ggml_new_tensor(ctx, type, 2, ne);
}
struct ggml_tensor *ggml_new_tensor_3d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0, int64_t ne1,
                                       int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return ggml_new_tensor(ctx, type, 3, ne);
}
struct ggml_tensor *ggml_new_tensor_4d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0, int64_t ne1,
                                       int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return ggml_new_tensor(ctx, type, 4, ne);
}

static ggml_tensor *dup_tensor(ggml_context *ctx, const ggml_tensor *a) {
    return ggml_new_tensor(ctx, a->type, GGML_MAX_DIMS, a->ne);
}

static ggml_tensor *view_tensor(ggml_context *ctx, ggml_tensor *a) {
    ggml_tensor *r = new_tensor_impl(ctx, a->type, GGML_MAX_DIMS, a->ne, a, 0);
    for (int i = 0; i < GGML_MAX_DIMS; i++) r->nb[i] = a->nb[i];
    snprintf(r->name, sizeof(r->name), "%.56s (view)", a->name);
    return r;
}

const char *ggml_get_name(const struct ggml_tensor *t) { return t->name; }

struct ggml_tensor *ggml_set_name(struct ggml_tensor *t, const char *name) {
    snprintf(t->name, sizeof(t->name), "%s", name);
    return t;
}

void ggml_set_input(struct ggml_tensor *t) { t->flags |= GGML_TENSOR_FLAG_INPUT; }
void ggml_set_output(struct ggml_tensor *t) { t->flags |= GGML_TENSOR_FLAG_OUTPUT; }

static void set_op_params(ggml_tensor *t, const void *p, size_t n) {
    GGML_ASSERT(n <= GGML_MAX_OP_PARAMS);
    memcpy(t->op_params, p, n);
}

// ---------------------------------------------------------------- views

struct ggml_tensor *ggml_reshape_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1) {
    GGML_ASSERT(ggml_is_contiguous(a) && ggml_nelements(a) == ne0 * ne1);
    const int64_t ne[2] = {ne0, ne1};
    ggml_tensor *r = new_tensor_impl(ctx, a->type, 2, ne, a, 0);
    snprintf(r->name, sizeof(r->name), "%.52s (reshaped)", a->name);
    r->op = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}

struct ggml_tensor *ggml_reshape_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                    int64_t ne2) {
    GGML_ASSERT(ggml_is_contiguous(a) && ggml_nelements(a) == ne0 * ne1 * ne2);
    const int64_t ne[3] = {ne0, ne1, ne2};
    ggml_tensor *r = new_tensor_impl(ctx, a->type, 3, ne, a, 0);
    snprintf(r->name, sizeof(r->name), "%.52s (reshaped)", a->name);
    r->op = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}

struct ggml_tensor *ggml_reshape_4d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                    int64_t ne2, int64_t ne3) {
    GGML_ASSERT(ggml_is_contiguous(a) && ggml_nelements(a) == ne0 * ne1 * ne2 * ne3);
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    ggml_tensor *r = new_tensor_impl(ctx, a->type, 4, ne, a, 0);
    snprintf(r->name, sizeof(r->name), "%.52s (reshaped)", a->name);
    r->op = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}

static ggml_tensor *view_impl(ggml_context *ctx, ggml_tensor *a, int n_dims, const int64_t *ne, size_t offset) {
    ggml_tensor *r = new_tensor_impl(ctx, a->type, n_dims, ne, a, offset);
    snprintf(r->name, sizeof(r->name), "%.56s (view)", a->name);
    set_op_params(r, &offset, sizeof(offset));
    r->op = GGML_OP_VIEW;
    r->src[0] = a;
    return r;
}

struct ggml_tensor *ggml_view_1d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, size_t offset) {
    return view_impl(ctx, a, 1, &ne0, offset);
}

struct ggml_tensor *ggml_view_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                 size_t nb1, size_t offset) {
    const int64_t ne[2] = {ne0, ne1};
    ggml_tensor *r = view_impl(ctx, a, 2, ne, offset);
    r->nb[1] = nb1;
    r->nb[2] = r->nb[1] * (size_t)ne1;
    r->nb[3] = r->nb[2];
    return r;
}

struct ggml_tensor *ggml_view_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                 int64_t ne2, size_t nb1, size_t nb2, size_t offset) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    ggml_tensor *r = view_impl(ctx, a, 3, ne, offset);
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = r->nb[2] * (size_t)ne2;
    return r;
}

struct ggml_tensor *ggml_view_4d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                 int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    ggml_tensor *r = view_impl(ctx, a, 4, ne, offset);
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = nb3;
    return r;
}

struct ggml_tensor *ggml_permute(struct ggml_context *ctx, struct ggml_tensor *a, int axis0, int axis1, int axis2,
                                 int axis3) {
    GGML_ASSERT(axis0 != axis1 && axis0 != axis2 && axis0 != axis3 && axis1 != axis2 && axis1 != axis3 &&
                axis2 != axis3);
    ggml_tensor *r = view_tensor(ctx, a);
    int64_t ne[4];
    size_t nb[4];
    ne[axis0] = a->ne[0]; ne[axis1] = a->ne[1]; ne[axis2] = a->ne[2]; ne[axis3] = a->ne[3];
    nb[axis0] = a->nb[0]; nb[axis1] = a->nb[1]; nb[axis2] = a->nb[2]; nb[axis3] = a->nb[3];
    for (int i = 0; i < 4; i++) {
        r->ne[i] = ne[i];
        r->nb[i] = nb[i];
    }
    snprintf(r->name, sizeof(r->name), "%.52s (permuted)", a->name);
    r->op = GGML_OP_PERMUTE;
    r->src[0] = a;
    const int32_t params[4] = {axis0, axis1, axis2, axis3};
    set_op_params(r, params, sizeof(params));
    return r;
}

// ---------------------------------------------------------------- ops

static bool can_repeat(const ggml_tensor *t0, const ggml_tensor *t1) {
    return (t1->ne[0] % t0->ne[0] == 0) && (t1->ne[1] % t0->ne[1] == 0) && (t1->ne[2] % t0->ne[2] == 0) &&
           (t1->ne[3] % t0->ne[3] == 0);
}

static ggml_tensor *binary(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b, ggml_op op) {
    GGML_ASSERT(can_repeat(b, a));
    ggml_tensor *r = dup_tensor(ctx, a);
    r->op = op;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor *ggml_add(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    return binary(ctx, a, b, GGML_OP_ADD);
}

struct ggml_tensor *ggml_mul(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    return binary(ctx, a, b, GGML_OP_MUL);
}

struct ggml_tensor *ggml_rms_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps) {
    ggml_tensor *r = dup_tensor(ctx, a);
    set_op_params(r, &eps, sizeof(eps));
    r->op = GGML_OP_RMS_NORM;
    r->src[0] = a;
    return r;
}

struct ggml_tensor *ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    GGML_ASSERT(a->ne[0] == b->ne[0] && b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0);
    const int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    ggml_tensor *r = ggml_new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    r->op = GGML_OP_MUL_MAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor *ggml_get_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    GGML_ASSERT(a->ne[2] == b->ne[1] && b->ne[3] == 1 && b->type == GGML_TYPE_I32);
    const ggml_type t = a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32;
    ggml_tensor *r = ggml_new_tensor_4d(ctx, t, a->ne[0], b->ne[0], b->ne[1], b->ne[2]);
    r->op = GGML_OP_GET_ROWS;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor *ggml_set_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                  struct ggml_tensor *c) {
    GGML_ASSERT(a->ne[0] == b->ne[0] && b->ne[1] == c->ne[0]);
    GGML_ASSERT(c->type == GGML_TYPE_I64 || c->type == GGML_TYPE_I32);
    ggml_tensor *r = view_tensor(ctx, a);
    r->op = GGML_OP_SET_ROWS;
    r->src[0] = b;
    r->src[1] = c;
    return r;
}

struct ggml_tensor *ggml_rope_ext(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                  struct ggml_tensor *c, int n_dims, int mode, int n_ctx_orig, float freq_base,
                                  float freq_scale, float ext_factor, float attn_factor, float beta_fast,
                                  float beta_slow) {
    GGML_ASSERT(b->type == GGML_TYPE_I32 && a->ne[2] == b->ne[0]);
    ggml_tensor *r = dup_tensor(ctx, a);
    int32_t params[15] = {0, n_dims, mode, 0, n_ctx_orig};
    memcpy(params + 5, &freq_base, sizeof(float));
    memcpy(params + 6, &freq_scale, sizeof(float));
    memcpy(params + 7, &ext_factor, sizeof(float));
    memcpy(params + 8, &attn_factor, sizeof(float));
    memcpy(params + 9, &beta_fast, sizeof(float));
    memcpy(params + 10, &beta_slow, sizeof(float));
    set_op_params(r, params, sizeof(params));
    r->op = GGML_OP_ROPE;
    r->src[0] = a;
    r->src[1] = b;
    r->src[2] = c;
    return r;
}

struct ggml_tensor *ggml_flash_attn_ext(struct ggml_context *ctx, struct ggml_tensor *q, struct ggml_tensor *k,
                                        struct ggml_tensor *v, struct ggml_tensor *mask, float scale, float max_bias,
                                        float logit_softcap) {
    GGML_ASSERT(q->ne[0] == k->ne[0] && k->ne[1] == v->ne[1]);
    if (mask) GGML_ASSERT(mask->ne[0] >= k->ne[1] && mask->ne[1] >= q->ne[1]);
    const int64_t ne[4] = {v->ne[0], q->ne[2], q->ne[1], q->ne[3]};
    ggml_tensor *r = ggml_new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    const float params[3] = {scale, max_bias, logit_softcap};
    set_op_params(r, params, sizeof(params));
    r->op = GGML_OP_FLASH_ATTN_EXT;
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->src[3] = mask;
    return r;
}

void ggml_flash_attn_ext_set_prec(struct ggml_tensor *a, enum ggml_prec prec) {
    GGML_ASSERT(a->op == GGML_OP_FLASH_ATTN_EXT);
    a->op_params[3] = (int32_t)prec;
}

void ggml_flash_attn_ext_add_kv_lengths(struct ggml_tensor *a, struct ggml_tensor *kv_lengths) {
    if (!kv_lengths) {
        a->src[5] = nullptr;
        return;
    }
    GGML_ASSERT(a->op == GGML_OP_FLASH_ATTN_EXT);
    GGML_ASSERT(a->src[5] == nullptr);
    GGML_ASSERT(kv_lengths->type == GGML_TYPE_I32);
    GGML_ASSERT(ggml_is_contiguous(kv_lengths));
    a->src[5] = kv_lengths;
}

struct ggml_tensor *ggml_swiglu_split(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    GGML_ASSERT(ggml_are_same_shape(a, b) && a->type == b->type);
    ggml_tensor *r = dup_tensor(ctx, a);
    const int32_t params[2] = {GGML_GLU_OP_SWIGLU, 0};
    set_op_params(r, params, sizeof(params));
    r->op = GGML_OP_GLU;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor *ggml_silu(struct ggml_context *ctx, struct ggml_tensor *a) {
    ggml_tensor *r = dup_tensor(ctx, a);
    const int32_t p = GGML_UNARY_OP_SILU;
    set_op_params(r, &p, sizeof(p));
    r->op = GGML_OP_UNARY;
    r->src[0] = a;
    return r;
}

struct ggml_tensor *ggml_argmax(struct ggml_context *ctx, struct ggml_tensor *a) {
    GGML_ASSERT(a->ne[2] == 1 && a->ne[3] == 1);
    ggml_tensor *r = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, a->ne[1]);
    r->op = GGML_OP_ARGMAX;
    r->src[0] = a;
    return r;
}

struct ggml_tensor *ggml_cpy(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    GGML_ASSERT(ggml_nelements(a) == ggml_nelements(b));
    ggml_tensor *r = view_tensor(ctx, b);
    r->op = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

// ---------------------------------------------------------------- graphs

struct ggml_cgraph *ggml_new_graph_custom(struct ggml_context *ctx, size_t size, bool grads) {
    (void)grads;
    ctx->graphs.emplace_back();
    ggml_cgraph *g = &ctx->graphs.back();
    g->size = (int)size;
    return g;
}

struct ggml_cgraph *ggml_new_graph(struct ggml_context *ctx) {
    return ggml_new_graph_custom(ctx, GGML_DEFAULT_GRAPH_SIZE, false);
}

static void visit(ggml_cgraph *g, ggml_tensor *t) {
    if (!t || g->visited.count(t)) return;
    g->visited.insert(t);
    for (int i = 0; i < GGML_MAX_SRC; i++) visit(g, t->src[i]);
    if (t->op == GGML_OP_NONE && !(t->flags & GGML_TENSOR_FLAG_PARAM)) {
        g->leafs.push_back(t);
    } else {
        GGML_ASSERT((int)g->nodes.size() < g->size);
        g->nodes.push_back(t);
    }
}

void ggml_build_forward_expand(struct ggml_cgraph *cgraph, struct ggml_tensor *tensor) { visit(cgraph, tensor); }

int ggml_graph_n_nodes(struct ggml_cgraph *g) { return (int)g->nodes.size(); }

struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *g, int i) {
    if (i < 0) i += (int)g->nodes.size();
    GGML_ASSERT(i >= 0 && i < (int)g->nodes.size());
    return g->nodes[i];
}

int ggml_graph_n_leafs(struct ggml_cgraph *g) { return (int)g->leafs.size(); }

struct ggml_tensor *ggml_graph_leaf(struct ggml_cgraph *g, int i) {
    GGML_ASSERT(i >= 0 && i < (int)g->leafs.size());
    return g->leafs[i];
}

}  // extern "C"

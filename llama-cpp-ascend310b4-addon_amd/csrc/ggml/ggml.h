/*
 * ggml.h -- the subset of ggml's public tensor/graph API (llama.cpp @ 37b3a9e0,
 * ggml/include/ggml.h) that the MI355X backend and its decode-graph driver use,
 * restated so that the backend builds and is testable without a llama.cpp tree.
 *
 * Names, member order of struct ggml_tensor, type ids and the semantics of
 * every function follow upstream ggml; the numeric values of enum ggml_op are
 * this file's own (the backend only compares against the names).  When the
 * backend is compiled inside a real llama.cpp tree this header is not used.
 */
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_API

#define GGML_MAX_DIMS 4
#define GGML_MAX_PARAMS 2048
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64
#define GGML_MAX_OP_PARAMS 64
#define GGML_DEFAULT_GRAPH_SIZE 2048
#define GGML_MEM_ALIGN 16

#define GGML_PAD(x, n) (((x) + (n) - 1) & ~((n) - 1))

#define GGML_ROPE_TYPE_NEOX 2

typedef uint16_t ggml_fp16_t;

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

/* type ids are upstream's (they are stored in GGUF files) */
enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q4_1 = 3,
    GGML_TYPE_Q5_0 = 6,
    GGML_TYPE_Q5_1 = 7,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_I8 = 24,
    GGML_TYPE_I16 = 25,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_I64 = 27,
    GGML_TYPE_F64 = 28,
    GGML_TYPE_BF16 = 30,
    GGML_TYPE_COUNT = 40,
};

enum ggml_prec {
    GGML_PREC_DEFAULT = 0,
    GGML_PREC_F32 = 10,
};

enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP,
    GGML_OP_ADD,
    GGML_OP_SUB,
    GGML_OP_MUL,
    GGML_OP_DIV,
    GGML_OP_ARGMAX,
    GGML_OP_RMS_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_SCALE,
    GGML_OP_CPY,
    GGML_OP_CONT,
    GGML_OP_RESHAPE,
    GGML_OP_VIEW,
    GGML_OP_PERMUTE,
    GGML_OP_TRANSPOSE,
    GGML_OP_GET_ROWS,
    GGML_OP_SET_ROWS,
    GGML_OP_SOFT_MAX,
    GGML_OP_ROPE,
    GGML_OP_FLASH_ATTN_EXT,
    GGML_OP_UNARY,
    GGML_OP_GLU,
    GGML_OP_COUNT,
};

enum ggml_unary_op {
    GGML_UNARY_OP_SILU = 10,
    GGML_UNARY_OP_COUNT = 16,
};

enum ggml_glu_op {
    GGML_GLU_OP_REGLU = 0,
    GGML_GLU_OP_GEGLU = 1,
    GGML_GLU_OP_SWIGLU = 2,
    GGML_GLU_OP_COUNT,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
    GGML_TENSOR_FLAG_PARAM = 4,
    GGML_TENSOR_FLAG_LOSS = 8,
};

struct ggml_backend_buffer;

struct ggml_tensor {
    enum ggml_type type;

    struct ggml_backend_buffer *buffer;

    int64_t ne[GGML_MAX_DIMS]; /* number of elements */
    size_t nb[GGML_MAX_DIMS];  /* stride in bytes */

    enum ggml_op op;

    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];

    int32_t flags;

    struct ggml_tensor *src[GGML_MAX_SRC];

    struct ggml_tensor *view_src;
    size_t view_offs;

    void *data;

    char name[GGML_MAX_NAME];

    void *extra; /* backend-specific data */

    char padding[8];
};

struct ggml_context;
struct ggml_cgraph;

struct ggml_init_params {
    size_t mem_size;   /* bytes for tensor data when !no_alloc (tensor headers are separate here) */
    void *mem_buffer;  /* unused: the context owns its memory */
    bool no_alloc;     /* true: tensors get no data (a backend buffer provides it) */
};

/* ---- types and sizes ---- */
GGML_API int64_t ggml_blck_size(enum ggml_type type);
GGML_API size_t ggml_type_size(enum ggml_type type);
GGML_API size_t ggml_row_size(enum ggml_type type, int64_t ne);
GGML_API const char *ggml_type_name(enum ggml_type type);
GGML_API const char *ggml_op_name(enum ggml_op op);
GGML_API bool ggml_is_quantized(enum ggml_type type);

GGML_API int64_t ggml_nelements(const struct ggml_tensor *tensor);
GGML_API int64_t ggml_nrows(const struct ggml_tensor *tensor);
GGML_API size_t ggml_nbytes(const struct ggml_tensor *tensor);
GGML_API bool ggml_is_contiguous(const struct ggml_tensor *tensor);
GGML_API bool ggml_is_empty(const struct ggml_tensor *tensor);
GGML_API bool ggml_are_same_shape(const struct ggml_tensor *t0, const struct ggml_tensor *t1);

GGML_API enum ggml_unary_op ggml_get_unary_op(const struct ggml_tensor *tensor);
GGML_API enum ggml_glu_op ggml_get_glu_op(const struct ggml_tensor *tensor);

/* ---- context ---- */
GGML_API struct ggml_context *ggml_init(struct ggml_init_params params);
GGML_API void ggml_free(struct ggml_context *ctx);
GGML_API bool ggml_get_no_alloc(struct ggml_context *ctx);
GGML_API struct ggml_tensor *ggml_get_first_tensor(const struct ggml_context *ctx);
GGML_API struct ggml_tensor *ggml_get_next_tensor(const struct ggml_context *ctx, struct ggml_tensor *tensor);
GGML_API struct ggml_tensor *ggml_get_tensor(struct ggml_context *ctx, const char *name);

GGML_API struct ggml_tensor *ggml_new_tensor(struct ggml_context *ctx, enum ggml_type type, int n_dims,
                                             const int64_t *ne);
GGML_API struct ggml_tensor *ggml_new_tensor_1d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0);
GGML_API struct ggml_tensor *ggml_new_tensor_2d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                int64_t ne1);
GGML_API struct ggml_tensor *ggml_new_tensor_3d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor *ggml_new_tensor_4d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                int64_t ne1, int64_t ne2, int64_t ne3);

GGML_API const char *ggml_get_name(const struct ggml_tensor *tensor);
GGML_API struct ggml_tensor *ggml_set_name(struct ggml_tensor *tensor, const char *name);
GGML_API void ggml_set_input(struct ggml_tensor *tensor);
GGML_API void ggml_set_output(struct ggml_tensor *tensor);

/* ---- views ---- */
GGML_API struct ggml_tensor *ggml_reshape_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                             int64_t ne1);
GGML_API struct ggml_tensor *ggml_reshape_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                             int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor *ggml_reshape_4d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                             int64_t ne1, int64_t ne2, int64_t ne3);
GGML_API struct ggml_tensor *ggml_view_1d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                          size_t offset);
GGML_API struct ggml_tensor *ggml_view_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                          size_t nb1, size_t offset);
GGML_API struct ggml_tensor *ggml_view_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                          int64_t ne2, size_t nb1, size_t nb2, size_t offset);
GGML_API struct ggml_tensor *ggml_view_4d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                          int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3,
                                          size_t offset);
GGML_API struct ggml_tensor *ggml_permute(struct ggml_context *ctx, struct ggml_tensor *a, int axis0, int axis1,
                                          int axis2, int axis3);

/* ---- ops (upstream semantics) ---- */
GGML_API struct ggml_tensor *ggml_add(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_mul(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_rms_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps);
/* a: [K, N] weight, b: [K, M] -> [N, M] */
GGML_API struct ggml_tensor *ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_get_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_set_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                           struct ggml_tensor *c);
GGML_API struct ggml_tensor *ggml_rope_ext(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                           struct ggml_tensor *c, int n_dims, int mode, int n_ctx_orig,
                                           float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                           float beta_fast, float beta_slow);
/* q: [D, n_q, n_head, 1] f32; k, v: [D, n_kv, n_head_kv, 1]; mask: [n_kv, n_q_pad] f16 or NULL
 * -> [D, n_head, n_q, 1] f32 */
GGML_API struct ggml_tensor *ggml_flash_attn_ext(struct ggml_context *ctx, struct ggml_tensor *q, struct ggml_tensor *k,
                                                 struct ggml_tensor *v, struct ggml_tensor *mask, float scale,
                                                 float max_bias, float logit_softcap);
GGML_API void ggml_flash_attn_ext_set_prec(struct ggml_tensor *a, enum ggml_prec prec);
/* optional I32 tensor with the effective KV boundary of each mask row (src[5]);
 * the reference's extension, patch:1020-1036, 2001-2024 */
GGML_API void ggml_flash_attn_ext_add_kv_lengths(struct ggml_tensor *a, struct ggml_tensor *kv_lengths);
GGML_API struct ggml_tensor *ggml_swiglu_split(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_silu(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_argmax(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_cpy(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);

/* ---- graphs ---- */
GGML_API struct ggml_cgraph *ggml_new_graph(struct ggml_context *ctx);
GGML_API struct ggml_cgraph *ggml_new_graph_custom(struct ggml_context *ctx, size_t size, bool grads);
GGML_API void ggml_build_forward_expand(struct ggml_cgraph *cgraph, struct ggml_tensor *tensor);
GGML_API int ggml_graph_n_nodes(struct ggml_cgraph *cgraph);
GGML_API struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *cgraph, int i); /* i < 0: from the end */
GGML_API int ggml_graph_n_leafs(struct ggml_cgraph *cgraph);
GGML_API struct ggml_tensor *ggml_graph_leaf(struct ggml_cgraph *cgraph, int i);

/* ---- fp16 ---- */
GGML_API float ggml_fp16_to_fp32(ggml_fp16_t h);
GGML_API ggml_fp16_t ggml_fp32_to_fp16(float f);

#define GGML_ASSERT(x)                                                             \
    do {                                                                           \
        if (!(x)) ggml_abort(__FILE__, __LINE__, "GGML_ASSERT(%s) failed", #x);   \
    } while (0)
#define GGML_ABORT(...) ggml_abort(__FILE__, __LINE__, __VA_ARGS__)
GGML_API [[noreturn]] void ggml_abort(const char *file, int line, const char *fmt, ...);

#ifdef __cplusplus
}
#endif

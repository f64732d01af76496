/*
 * ggml-mi355x.h -- public entry points of the MI355X ggml backend.
 *
 * The backend plugs into llama.cpp's existing ggml_backend / ggml_backend_buffer_type
 * API exactly where the CANN backend does (ggml/include/ggml-cann.h of llama.cpp @
 * 37b3a9e0: ggml_backend_cann_init / _is_cann / _buffer_type / _get_device_count /
 * _get_device_description / _get_device_memory / _reg), so the scheduler's
 * supports_op routing, the loader's set_tensor / get_alloc_size calls and
 * graph_compute reach it unchanged.  What changes behind that API for the decode
 * hot path (the 310B branch of ggml-cann, patch:1037-1986):
 *   - buffer get_alloc_size / set_tensor: Q8_0 and Q4_0 matmul weights get a
 *     planar side copy after the ggml bytes (replaces the FRACTAL_NZ / INT8-NZ side
 *     copies of patch:1535-1562, 1700-1847); F16 weights, including the tied output
 *     head, stream from their ND rows (no dual layout, patch:1451-1464);
 *   - MUL_MAT (M <= 8) runs the A8W8 / W4A16 / F16 GEMV kernels (patch:1188-1355);
 *   - FLASH_ATTN_EXT with one query row runs split-KV GQA flash-decoding for
 *     head dims 64 and 128 and honours the I32 kv_lengths src[5]
 *     (patch:1370-1442, 1957-1983, 2001-2024).
 */
#pragma once

#include "ggml.h"
#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef GGML_BACKEND_API
#define GGML_BACKEND_API
#endif

#define GGML_MI355X_NAME "MI355X"
#define GGML_MI355X_MAX_DEVICES 16

/* backend for one HIP device (one stream); NULL when the device does not exist */
GGML_BACKEND_API ggml_backend_t ggml_backend_mi355x_init(int device);
GGML_BACKEND_API bool ggml_backend_is_mi355x(ggml_backend_t backend);
/* device memory buffer type; weight tensors uploaded through it are prepacked */
GGML_BACKEND_API ggml_backend_buffer_type_t ggml_backend_mi355x_buffer_type(int device);
GGML_BACKEND_API int ggml_backend_mi355x_get_device_count(void);
GGML_BACKEND_API void ggml_backend_mi355x_get_device_description(int device, char *description,
                                                                 size_t description_size);
GGML_BACKEND_API void ggml_backend_mi355x_get_device_memory(int device, size_t *free, size_t *total);
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_mi355x_reg(void);

/* SmoothQuant: the Q8_0 weight holds W*diag(s); MUL_MAT with this weight quantizes x/s
 * (x times the fp32 reciprocal of s).  Tensors sharing one s pointer of equal content
 * share the device copy.  The reference reads no scale file at run time (its interface
 * is described in tools/smoothquant/README.md); this is the runtime side of that
 * contract.  Returns false if the tensor is not a prepacked Q8_0 weight of this backend
 * or n != ne[0]. */
GGML_BACKEND_API bool ggml_backend_mi355x_set_smooth_factors(struct ggml_tensor *weight, const float *s, int64_t n);

#ifdef __cplusplus
}
#endif

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
 *     copies of patch:1535-1562, 1700-1847); with GGML_MI355X_A8W8=1, F16 projection
 *     weights get a Q8_0 side copy quantized on the device (patch:1472-1533,
 *     1674-1751; GGML_MI355X_A8W8_DISABLE_LAYERS keeps listed layers F16); other F16
 *     weights, including the tied output head, stream from their ND rows (no dual
 *     layout, patch:1451-1464);
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

/* SmoothQuant factors s[n] (n = ne[0], every s > 0 and finite) of one projection weight:
 * MUL_MAT with this weight quantizes x/s (x times the fp32 reciprocal of s) against a
 * Q8_0 weight that holds W*diag(s).
 *   - F16 weight on the A8W8 path (GGML_MI355X_A8W8=1, quantized at upload, the
 *     reference's GGML_CANN_A8W8 of patch:1472-1533): the backend folds s in itself,
 *     re-quantizing W*diag(s) to Q8_0 on the device from the F16 bytes it keeps.
 *   - Q8_0 weight: only the activation divisor is set; the blocks must already hold
 *     W*diag(s) (quantized offline from the smoothed weight).
 *   - F16 weight without a Q8_0 copy (a layer GGML_MI355X_A8W8_DISABLE_LAYERS keeps F16,
 *     or A8W8 off): accepted, nothing changes, since (x/s) . W*diag(s) = W.x exactly.
 * Tensors given equal factors share one device copy.  Returns false, changing nothing,
 * for a weight of another backend's buffer, a W4A16 (Q4_0) weight, n != ne[0], or a
 * factor that is not a positive finite number.  The reference reads the
 * scale file of tools/smoothquant/smoothquant-make-scales.py:14-17 offline; this is the
 * runtime side of that contract. */
GGML_BACKEND_API bool ggml_backend_mi355x_set_smooth_factors(struct ggml_tensor *weight, const float *s, int64_t n);

/* No counterpart in the reference (the persistent layer-stack decode, GGML_MI355X_PERSIST=1,
 * has in-kernel dependency waits that give up after a bounded number of polls): waits for
 * the backend's stream, then returns 0, or -1 when a launch since the last call gave up
 * (its results are invalid; the next graph_compute also reports GGML_STATUS_FAILED once). */
GGML_BACKEND_API int ggml_backend_mi355x_status(ggml_backend_t backend);
/* With GGML_MI355X_PERSIST_TIMING=1 set when the backend was created: the number of
 * persistent layer-stack launches timed so far and their summed duration in ms (HIP
 * events on the backend's stream around each launch run eagerly, i.e. not inside a
 * captured graph; read at each ggml_backend_mi355x_status).  Returns 0, or -1 when the
 * timing is off.  No reference counterpart (a measurement hook). */
GGML_BACKEND_API int ggml_backend_mi355x_persist_timing(ggml_backend_t backend, int64_t *launches, double *total_ms);

/* No counterpart in the reference (an integration check for dynamic loading): returns 1
 * when the op and type ids this backend was compiled with carry the same names in the
 * loaded ggml (ggml_op_name / ggml_type_name), else 0; msg receives a description.
 * ggml_backend_init (GGML_BACKEND_DL builds) refuses to register on a mismatch. */
GGML_BACKEND_API int ggml_backend_mi355x_abi_check(char *msg, size_t msg_size);

#ifdef __cplusplus
}
#endif

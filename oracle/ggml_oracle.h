/*
 * ggml_oracle.h -- CPU restatement of the ggml-CPU semantics on the
 * single-token decode path (Q8_0 / Q4_0 / F16 mul_mat at M=1 and
 * single-token flash_attn_ext), used ONLY as the test checker and as the
 * timed CPU baseline.  Nothing in the product library links or calls this.
 *
 * The algorithms restated here live in upstream llama.cpp/ggml
 * (https://github.com/ggml-org/llama.cpp.git @ 37b3a9e0ccba261d1cc245a971deae0b18c201ab,
 * the base commit named by the reference at manifest.json:4 and
 * scripts/install.sh:5).  That tree is a third-party dependency that is not
 * vendored in the reference and not present offline, so each function
 * restates the published algorithm and names the upstream function it follows:
 *
 *   ggml/src/ggml-quants.c        quantize_row_q8_0_ref, dequantize_row_q4_0
 *   ggml/src/ggml-cpu/arch/x86/quants.c  quantize_row_q8_0 (AVX path),
 *                                 ggml_vec_dot_q8_0_q8_0
 *   ggml/src/ggml-cpu/vec.h/.cpp  ggml_vec_dot_f16, ggml_vec_mad_f16,
 *                                 ggml_vec_scale_f16
 *   ggml/src/ggml-cpu/ops.cpp     ggml_compute_forward_flash_attn_ext_f16
 *
 * Reference-side anchors (paths relative to the reference repository):
 *   patch:1674-1695   per-channel A8W8 weight quant (restated: orc_quantize_a8w8_per_channel)
 *   experiments/a8w8/w8a8_quantize_custom_vector.cpp:28-57 per-token act quant
 *                     (restated: orc_quantize_per_token_i8)
 *   experiments/a8w8/custom_a8w8_chain_probe.cpp:104-115,189 and
 *   experiments/a8w8/quant_matmul_v3_probe.cpp:30-32,76-77  known answers
 *   experiments/w4a16-gemv/source/w4a16_gemv_qwen.cpp:127-148 nibble offset 8,
 *                     group scale applied after the group sum
 *   experiments/attention-step-custom/custom_ops/op_kernel/attention_step_custom.cpp:109-277
 *                     decode attention order (scale, mask, online softmax, final divide)
 *   patch:2900-2929   kv_lengths derivation from the mask
 *
 * Parity status of each function is listed in the test module
 * tests/test_oracle.py; a function with no independent check there is
 * marked "parity unpinned" in its comment below.
 */
#ifndef GGML_ORACLE_H
#define GGML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK8_0 32
#define ORC_QK4_0 32

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[ORC_QK8_0]; } orc_block_q8_0;      /* 34 B, ggml block_q8_0 */
typedef struct { uint16_t d; uint8_t qs[ORC_QK4_0 / 2]; } orc_block_q4_0; /* 18 B, ggml block_q4_0 */
#pragma pack(pop)

/* rounding variants of the activation quantizer */
#define ORC_Q8_ROUND_REF 0  /* quantize_row_q8_0_ref: id = 1/d, roundf (half away from zero) */
#define ORC_Q8_ROUND_X86 1  /* ggml-cpu x86 AVX path: id = 127/amax, round-half-even */

/* ---- fp16 ---- */
uint16_t orc_fp32_to_fp16(float f);  /* IEEE binary16, round to nearest even */
float    orc_fp16_to_fp32(uint16_t h);
void     orc_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n);
void     orc_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n);

/* ---- Q8_0 ---- */
/* x (optionally multiplied element-wise by inv_s first) -> Q8_0 blocks */
void orc_quantize_row_q8_0(const float *x, const float *inv_s, orc_block_q8_0 *y, int64_t k, int variant);
void orc_dequantize_row_q8_0(const orc_block_q8_0 *x, float *y, int64_t k);
/* scalar ggml_vec_dot_q8_0_q8_0 (generic order) */
float orc_vec_dot_q8_0_q8_0(int64_t k, const orc_block_q8_0 *x, const orc_block_q8_0 *y);
/* exact per-block int32 dot products: out[n*nb + b] */
void orc_q8_0_block_dots(const orc_block_q8_0 *w, const orc_block_q8_0 *xq, int64_t n_rows, int64_t k, int32_t *out);
/* y[n] = W[n,:] . quant(x * inv_s), scalar checker */
void orc_mul_mat_q8_0(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                      int64_t n_rows, int64_t k, int variant);
/* same, M rows of activations (x: [m][k], y: [m][n_rows]) */
void orc_mul_mat_q8_0_batch(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                            int64_t n_rows, int64_t k, int64_t m, int variant);
/* host weight quantizer: W (fp32 [n][k]) * diag(s) -> Q8_0 (ggml ref rounding) */
void orc_quantize_weight_q8_0(const float *w, const float *s, orc_block_q8_0 *y, int64_t n_rows, int64_t k);

/* ---- Q4_0 ---- */
void orc_dequantize_row_q4_0(const orc_block_q4_0 *x, float *y, int64_t k);
/* y[n] = dequant(W[n,:]) . fp32(x_f16), fp32 accumulation in index order */
void orc_mul_mat_q4_0_f16(const orc_block_q4_0 *w, const uint16_t *x_f16, float *y, int64_t n_rows, int64_t k);
/* same in fp64 (tolerance anchor) */
void orc_mul_mat_q4_0_f16_f64(const orc_block_q4_0 *w, const uint16_t *x_f16, double *y, int64_t n_rows, int64_t k);

/* ---- F16 ---- */
/* ggml F16 mul_mat: src1 converted to fp16 (vec_dot_type), fp32 accumulation */
void orc_mul_mat_f16(const uint16_t *w, const float *x, float *y, int64_t n_rows, int64_t k);
void orc_mul_mat_f16_f64(const uint16_t *w, const float *x, double *y, int64_t n_rows, int64_t k);

/* ---- flash_attn_ext, one query token ---- */
/*
 * q    : fp32 [n_q_heads][d]
 * k, v : fp16, element (pos, head, i) at byte offset pos*nb1 + head*nb2 + i*2
 * mask : fp16 [n_kv] or NULL
 * kv_len: number of leading positions considered (<= n_kv)
 * out  : fp32 [n_q_heads][d]
 * mode : 0 = ggml-CPU faithful (q -> fp16, fp16 V accumulator),
 *        1 = fp64 textbook softmax attention on the same fp16-rounded q (exact answer)
 */
void orc_flash_attn_ext_1tok(const float *q, const void *k, const void *v, const uint16_t *mask,
                             int64_t kv_len, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                             size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale,
                             float *out, int mode);

/* ---- kv_lengths (patch:2900-2929) ---- */
void orc_kv_lengths(const void *mask, int mask_is_f16, int64_t n_kv, int64_t n_rows, int32_t *out);

/* ---- reference-side A8W8 scheme (patch:1674-1695, w8a8_quantize_custom_vector.cpp:28-57) ---- */
void orc_quantize_a8w8_per_channel(const uint16_t *w_f16, int64_t k, int64_t n, int8_t *q_nz, uint16_t *scales);
void orc_quantize_per_token_i8(const uint16_t *x_f16, int64_t k, int8_t *xq, uint16_t *scale);

/* ---- timed CPU baseline: multithreaded SIMD restatement of ggml-CPU ---- */
/* returns the SIMD ISA name used ("avx512vnni", "avx2", "scalar") */
const char *orc_simd_isa(void);
void orc_mul_mat_q8_0_mt(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                         int64_t n_rows, int64_t k, int n_threads);
/* same with the activation quantized by `variant` (ORC_Q8_ROUND_REF / ORC_Q8_ROUND_X86) */
void orc_mul_mat_q8_0_mt_variant(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                                 int64_t n_rows, int64_t k, int n_threads, int variant);
void orc_mul_mat_q4_0_f16_mt(const orc_block_q4_0 *w, const uint16_t *x_f16, float *y,
                             int64_t n_rows, int64_t k, int n_threads);
void orc_mul_mat_f16_mt(const uint16_t *w, const float *x, float *y, int64_t n_rows, int64_t k, int n_threads);
void orc_flash_attn_ext_1tok_mt(const float *q, const void *k, const void *v, const uint16_t *mask,
                                int64_t kv_len, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                                size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale,
                                float *out, int n_threads);

#ifdef __cplusplus
}
#endif
#endif

/*
 * qwen2_oracle.h -- CPU restatement of a llama.cpp Qwen2 decode step (TEST
 * INFRASTRUCTURE: the whole-model checker and CPU baseline).  See qwen2_oracle.c.
 */
#ifndef QWEN2_ORACLE_H
#define QWEN2_ORACLE_H

#include "ggml_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const float *attn_norm, *ffn_norm;                 /* [n_embd] */
    const void *wq, *wk, *wv, *wo, *wgate, *wup, *wdown; /* ggml Q8_0 / Q4_0 rows */
    const float *bq, *bk, *bv;                         /* biases or NULL */
    /* SmoothQuant reciprocals of each projection input (NULL = none):
     * q/k/v share one, o one, gate/up one, down one */
    const float *inv_s_attn, *inv_s_o, *inv_s_ffn, *inv_s_down;
} orc_qwen2_layer;

typedef struct {
    int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx;
    float rms_eps, rope_theta;
    int wtype;      /* 8 = Q8_0, 2 = Q4_0 */
    int fa_mode;    /* 0 = ggml-CPU faithful attention, 1 = fp64 */
    int n_threads;
    const uint16_t *tok_embd;   /* [n_vocab][n_embd] fp16, also the tied head */
    const float *output_norm;   /* [n_embd] */
    const orc_qwen2_layer *layers;
    uint16_t *k_cache, *v_cache; /* [n_layer][n_ctx][n_head_kv*head_dim] fp16 */
    int q8_variant; /* activation rounding of Q8_0 projections: ORC_Q8_ROUND_X86 (ggml-cpu on x86) or _REF */
    int q8_generic; /* 1: Q8_0 dots in ggml's generic (non-SIMD) summation order instead of AVX2/VNNI's */
} orc_qwen2;

/* one token at position pos (the cache holds positions < pos); logits [n_vocab]; returns the argmax */
int orc_qwen2_decode(const orc_qwen2 *m, int token, int pos, float *logits);

#ifdef __cplusplus
}
#endif
#endif

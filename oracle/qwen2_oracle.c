/*
 * qwen2_oracle.c -- CPU restatement of one llama.cpp Qwen2 decode step with
 * ggml-CPU op semantics (TEST INFRASTRUCTURE: whole-model checker and CPU
 * baseline; never linked by the product).
 *
 * Graph restated (llama.cpp @ 37b3a9e0, src/models/qwen2.cpp, not in the
 * reference tree): token_embd GET_ROWS -> per layer RMS_NORM*attn_norm, q/k/v
 * projections (+bias), neox RoPE (theta = pos * powf(base, -2/n_dims)^i by
 * repeated multiplication, ggml_rope_cache_init), fp16 KV cache write,
 * single-token flash_attn_ext, o projection, residual, RMS_NORM*ffn_norm,
 * gate/up, silu(gate)*up, down, residual -> RMS_NORM*output_norm -> tied fp16
 * head -> argmax (first maximum).  RMS_NORM sums x*x in double
 * (ggml_compute_forward_rms_norm_f32).  Q8_0 projections quantize the
 * activation (times the SmoothQuant reciprocal when given) with the x86 ggml-cpu
 * rounding (or the portable ggml reference rounding, q8_variant), summed in
 * the AVX2/VNNI order or, with q8_generic, in ggml's generic per-block order; Q4_0 projections use dequantize-then-fp32-dot on fp16 activations.
 * The reference's only model-level anchors are its greedy byte-compare gates
 * (patch:433, 617-621, 707-712), which need a real checkpoint: the per-op
 * functions this file composes are the ones pinned in tests/test_oracle.py.
 */
#include "qwen2_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static void rms_norm_mul(const float *x, const float *w, float *y, int n, float eps) {
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) y[i] = (x[i] * scale) * w[i];
}

static void rope_neox(float *x, int n_heads, int hd, int pos, float theta_base) {
    const float theta_scale = powf(theta_base, -2.0f / (float)hd);
    float cs[512][2];
    float theta = (float)pos;
    for (int i = 0; i < hd / 2; i++) {
        cs[i][0] = cosf(theta);
        cs[i][1] = sinf(theta);
        theta *= theta_scale;
    }
    for (int h = 0; h < n_heads; h++) {
        float *r = x + (size_t)h * hd;
        for (int i = 0; i < hd / 2; i++) {
            const float x0 = r[i], x1 = r[i + hd / 2];
            r[i] = x0 * cs[i][0] - x1 * cs[i][1];
            r[i + hd / 2] = x0 * cs[i][1] + x1 * cs[i][0];
        }
    }
}

static void proj(const orc_qwen2 *m, const void *w, const float *inv_s, const float *x, float *y, int n, int k) {
    if (m->wtype == 8 && m->q8_generic) {
        const int nb = k / ORC_QK8_0;
        orc_block_q8_0 *xq = (orc_block_q8_0 *)malloc((size_t)nb * sizeof(orc_block_q8_0));
        orc_quantize_row_q8_0(x, inv_s, xq, k, m->q8_variant);
#pragma omp parallel for num_threads(m->n_threads) schedule(static)
        for (int r = 0; r < n; r++) y[r] = orc_vec_dot_q8_0_q8_0(k, (const orc_block_q8_0 *)w + (size_t)r * nb, xq);
        free(xq);
    } else if (m->wtype == 8) {
        orc_mul_mat_q8_0_mt_variant((const orc_block_q8_0 *)w, x, inv_s, y, n, k, m->n_threads, m->q8_variant);
    } else {
        uint16_t *xh = (uint16_t *)malloc((size_t)k * 2);
        orc_fp32_to_fp16_row(x, xh, k);
        orc_mul_mat_q4_0_f16_mt((const orc_block_q4_0 *)w, xh, y, n, k, m->n_threads);
        free(xh);
    }
}

int orc_qwen2_decode(const orc_qwen2 *m, int token, int pos, float *logits) {
    const int E = m->n_embd, hd = m->head_dim, nkv = m->n_head_kv * hd, F = m->n_ff;
    float *x = (float *)malloc((size_t)E * 4), *cur = (float *)malloc((size_t)E * 4);
    float *q = (float *)malloc((size_t)E * 4), *kk = (float *)malloc((size_t)nkv * 4);
    float *vv = (float *)malloc((size_t)nkv * 4), *att = (float *)malloc((size_t)E * 4);
    float *g = (float *)malloc((size_t)F * 4), *u = (float *)malloc((size_t)F * 4);
    float *o = (float *)malloc((size_t)E * 4);
    orc_fp16_to_fp32_row(m->tok_embd + (size_t)token * E, x, E);
    for (int il = 0; il < m->n_layer; il++) {
        const orc_qwen2_layer *L = &m->layers[il];
        rms_norm_mul(x, L->attn_norm, cur, E, m->rms_eps);
        proj(m, L->wq, L->inv_s_attn, cur, q, E, E);
        proj(m, L->wk, L->inv_s_attn, cur, kk, nkv, E);
        proj(m, L->wv, L->inv_s_attn, cur, vv, nkv, E);
        if (L->bq) {
            for (int i = 0; i < E; i++) q[i] += L->bq[i];
            for (int i = 0; i < nkv; i++) kk[i] += L->bk[i];
            for (int i = 0; i < nkv; i++) vv[i] += L->bv[i];
        }
        rope_neox(q, m->n_head, hd, pos, m->rope_theta);
        rope_neox(kk, m->n_head_kv, hd, pos, m->rope_theta);
        uint16_t *kc = m->k_cache + (size_t)il * m->n_ctx * nkv;
        uint16_t *vc = m->v_cache + (size_t)il * m->n_ctx * nkv;
        orc_fp32_to_fp16_row(kk, kc + (size_t)pos * nkv, nkv);
        orc_fp32_to_fp16_row(vv, vc + (size_t)pos * nkv, nkv);
        const size_t nb1 = (size_t)nkv * 2, nb2 = (size_t)hd * 2;
        if (m->fa_mode == 0 && m->n_threads > 1)
            orc_flash_attn_ext_1tok_mt(q, kc, vc, NULL, pos + 1, m->n_head, m->n_head_kv, hd, nb1, nb2, nb1, nb2,
                                       1.0f / sqrtf((float)hd), att, m->n_threads);
        else
            orc_flash_attn_ext_1tok(q, kc, vc, NULL, pos + 1, m->n_head, m->n_head_kv, hd, nb1, nb2, nb1, nb2,
                                    1.0f / sqrtf((float)hd), att, m->fa_mode);
        proj(m, L->wo, L->inv_s_o, att, o, E, E);
        for (int i = 0; i < E; i++) x[i] = o[i] + x[i];
        rms_norm_mul(x, L->ffn_norm, cur, E, m->rms_eps);
        proj(m, L->wgate, L->inv_s_ffn, cur, g, F, E);
        proj(m, L->wup, L->inv_s_ffn, cur, u, F, E);
        for (int i = 0; i < F; i++) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
        proj(m, L->wdown, L->inv_s_down, g, o, E, F);
        for (int i = 0; i < E; i++) x[i] = o[i] + x[i];
    }
    rms_norm_mul(x, m->output_norm, cur, E, m->rms_eps);
    orc_mul_mat_f16_mt(m->tok_embd, cur, logits, m->n_vocab, E, m->n_threads);
    int best = 0;
    for (int i = 1; i < m->n_vocab; i++)
        if (logits[i] > logits[best]) best = i;
    free(x); free(cur); free(q); free(kk); free(vv); free(att); free(g); free(u); free(o);
    return best;
}

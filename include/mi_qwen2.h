/*
 * mi_qwen2.h -- a minimal Qwen2 decode driver over the ggml backend API.
 *
 * It stands in for the llama.cpp layers above the backend (model loader and
 * graph builder, src/llama-model.cpp / llama-graph.cpp of llama.cpp @ 37b3a9e0),
 * which are not part of this repository: it names tensors as llama.cpp's GGUF
 * loader does, uploads them with ggml_backend_tensor_set (so the backend's
 * prepack runs as it would under llama.cpp), builds the per-token graph with the
 * same nodes as llama.cpp's Qwen2 builder (RMS_NORM, MUL, MUL_MAT, ADD, ROPE neox,
 * SET_ROWS into an fp16 KV cache, FLASH_ATTN_EXT with the kv_lengths src[5] of
 * patch:2934-2997, GLU swiglu, GET_ROWS, ARGMAX) and runs it with
 * ggml_backend_graph_compute.  Each step decodes one token for each of n_seq independent
 * sequences (bs = n_seq; each sequence owns n_ctx cache positions), greedy sampling.
 */
#ifndef MI_QWEN2_H
#define MI_QWEN2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mi_qwen2_hparams {
    int32_t n_layer;
    int32_t n_embd;
    int32_t n_head;
    int32_t n_head_kv;
    int32_t head_dim;
    int32_t n_ff;
    int32_t n_vocab;
    int32_t n_ctx;      /* KV cache capacity (positions) */
    float rms_eps;
    float rope_theta;
    int32_t wtype;      /* ggml type id of the projection weights: 8 = Q8_0, 2 = Q4_0, 1 = F16 (A8W8 when the
                         * backend runs with GGML_MI355X_A8W8=1: quantized to Q8_0 at upload, else F16 GEMVs) */
    int32_t use_bias;   /* q/k/v biases (Qwen2 has them) */
    int32_t n_seq;      /* independent sequences decoded together, 1..8 (0 = 1) */
} mi_qwen2_hparams;

typedef struct mi_qwen2 mi_qwen2;

/* model with uninitialised weights and a zeroed KV cache on HIP device `device` */
mi_qwen2 *mi_qwen2_create(const mi_qwen2_hparams *hp, int device);
void mi_qwen2_free(mi_qwen2 *m);
const char *mi_qwen2_last_error(void);

/* upload one tensor by its GGUF name (token_embd.weight, blk.N.attn_q.weight, ...,
 * output_norm.weight); size must equal the tensor's ggml byte size */
int mi_qwen2_set_tensor(mi_qwen2 *m, const char *name, const void *data, size_t size);
/* SmoothQuant factors s (length = the weight's input dim) of one projection weight */
int mi_qwen2_set_smooth(mi_qwen2 *m, const char *weight_name, const float *s, int64_t n);
/* Read a SmoothQuant scale file: little-endian fp32 [n_layer][n_embd], every factor
 * positive and finite, the file's size exactly n_layer*n_embd*4 bytes.  The format is
 * the one tools/smoothquant/smoothquant-make-scales.py:14-17 writes (sq-scales-aXX.bin:
 * per layer the FFN input channels' s = a^alpha / w^(1-alpha), clipped to [1e-3, 1e3]).
 * Host-only; needs no device. */
int mi_smooth_scales_read(const char *path, int64_t n_layer, int64_t n_embd, float *out);
/* Load such a file into the model: row il is the SmoothQuant factor of blk.il.ffn_gate and
 * blk.il.ffn_up (mi_qwen2_set_smooth on each).  F16 weights on the A8W8 path get s folded
 * in by the backend (W*diag(s) quantized on the device).  Q8_0 weights must already hold
 * W*diag(s); the call refuses them unless weights_presmoothed != 0 asserts that. */
int mi_qwen2_load_smooth_file(mi_qwen2 *m, const char *path, int weights_presmoothed);
/* on != 0: later decode steps keep each layer's normed FFN input (ffn_norm-<layer>, the
 * input smoothquant-collect.py:15 reads) and FFN output (ffn_out-<layer>) as graph outputs,
 * so mi_qwen2_dump_layers can write them; the fused launches that would skip writing them
 * give way to unfused ones for those tensors. */
int mi_qwen2_set_layer_dump(mi_qwen2 *m, int on);
/* Write the latest decode step's layer tensors as LLDUMP1 records, the layer-dump format of
 * the reference's llama-eval-callback (patch:825-892, enabled there by LLAMA_LAYER_DUMP,
 * patch:928): the 8-byte magic "LLDUMP1\0" once, then per tensor a u16 name length, the
 * name, a u64 value count and the values as fp32, all little-endian.  Per layer, in graph
 * order: ffn_norm-<layer> and ffn_out-<layer> when the layer dump is on
 * (mi_qwen2_set_layer_dump), then l_out-<layer> (the residual stream after the layer);
 * each [n_embd, n_seq] fp32.  append != 0 appends to an existing dump (the header is
 * written when the file is empty). */
int mi_qwen2_dump_layers(mi_qwen2 *m, const char *path, int append);
/* byte size and dims of a named tensor (dims[0] = ne0, dims[1] = ne1); -1 if unknown */
int64_t mi_qwen2_tensor_nbytes(mi_qwen2 *m, const char *name, int64_t *dims);

int32_t mi_qwen2_n_seq(const mi_qwen2 *m);

/* one decode step at position pos (n_seq == 1): writes the argmax token, optionally the logits [n_vocab] */
int mi_qwen2_decode(mi_qwen2 *m, int32_t token, int32_t pos, int32_t *next_token, float *logits);
/* one decode step of all n_seq sequences: tokens[s] at position pos[s]; writes next_tokens[n_seq]
 * and optionally logits [n_seq][n_vocab] */
int mi_qwen2_decode_batch(mi_qwen2 *m, const int32_t *tokens, const int32_t *pos, int32_t *next_tokens,
                          float *logits);
/* n_steps greedy steps of all sequences from tokens[s] at pos[s]; out_tokens [n_steps][n_seq] */
int mi_qwen2_decode_steps_batch(mi_qwen2 *m, const int32_t *tokens, const int32_t *pos, int32_t n_steps,
                                int32_t *out_tokens, double *seconds);
/* prompt tokens of sequence seq at positions pos0.. in ubatches of up to n_ubatch (1..8)
 * tokens, one graph per ubatch as llama.cpp builds it for a prompt batch: MUL_MATs of
 * n_ubatch rows, FLASH_ATTN_EXT with n_ubatch query rows under the causal KQ mask (one F16
 * row per token) beside the kv length, logits of the ubatch's last token only.  Writes the
 * greedy token after the last prompt token (next_token) and its logits [n_vocab] when not
 * NULL, and the seconds taken.  Cf. the reference's prompt path, which feeds its ubatches
 * through the same graph (patch:940-1019 chunks the prompt; patch:1286-1309 routes any M). */
int mi_qwen2_prefill(mi_qwen2 *m, int32_t seq, const int32_t *tokens, int32_t n_tokens, int32_t pos0,
                     int32_t n_ubatch, int32_t *next_token, float *logits, double *seconds);
/* the prompt (one token per step), then n_gen timed greedy decode steps: the first
 * consumes the prompt's greedy continuation, out_tokens[i] is the token step i produces;
 * the seconds of the n_gen steps are written to *gen_seconds when not NULL */
int mi_qwen2_generate(mi_qwen2 *m, const int32_t *prompt, int32_t n_prompt, int32_t n_gen, int32_t *out_tokens,
                      double *gen_seconds);
/* n_steps greedy decode steps continuing from `token` at position `pos` (the cache holds
 * positions < pos): step i feeds the previous step's argmax and writes it to out_tokens[i];
 * the wall-clock seconds of the n_steps are written to *seconds when not NULL */
int mi_qwen2_decode_steps(mi_qwen2 *m, int32_t token, int32_t pos, int32_t n_steps, int32_t *out_tokens,
                          double *seconds);
/* copy the first n_pos positions of layer `layer`'s K (is_v = 0) or V (is_v = 1) cache,
 * fp16 [n_pos][n_head_kv*head_dim], into host memory dst of `size` bytes (the state a
 * llama.cpp session save would write for this sequence) */
int mi_qwen2_get_cache(mi_qwen2 *m, int32_t layer, int32_t is_v, int32_t n_pos, void *dst, size_t size);
/* the same for sequence seq, and its inverse (the state a session load would restore) */
int mi_qwen2_get_cache_seq(mi_qwen2 *m, int32_t layer, int32_t is_v, int32_t seq, int32_t n_pos, void *dst,
                           size_t size);
int mi_qwen2_set_cache_seq(mi_qwen2 *m, int32_t layer, int32_t is_v, int32_t seq, int32_t n_pos, const void *src,
                           size_t size);
/* the backend's persistent-launch timing (ggml_backend_mi355x_persist_timing): launches
 * timed so far and their summed ms; -1 unless GGML_MI355X_PERSIST_TIMING=1 was set when the
 * model was created */
int mi_qwen2_persist_timing(mi_qwen2 *m, int64_t *launches, double *total_ms);
/* synthetic context: positions < n_pos of every layer's K and V cache of every sequence set to
 * fp16 values uniform in [-scale, scale) on the device (decode timing at long contexts) */
int mi_qwen2_fill_cache(mi_qwen2 *m, int32_t n_pos, uint64_t seed, float scale);
/* forget the KV cache contents (positions restart at 0) */
int mi_qwen2_reset(mi_qwen2 *m);

#ifdef __cplusplus
}
#endif
#endif
